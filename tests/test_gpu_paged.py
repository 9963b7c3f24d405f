"""Parity of the paged fp8 / bf16 kernels with the oracle on the GPU.

* append: fp8 codes bit-exact against the oracle's ``fp8_encode`` (techniques/kv_quant/fp8.py:81-86) at every slot;
  per-head scales bit-exact against ``static_scales`` (fp8.py:130-133).
* decode: within atol 2e-3 / rtol 1e-2 of the fp32 definition (attention/decode.py:66-103) over the gathered,
  decoded cache, for GQA shapes, ragged and empty rows, verification queries (causal), soft caps and sinks.
* every finite fp8 byte decodes exactly (the reference's test_fp8_bytes_decode_exactly,
  tests/unit/test_attention_kernel.py:146-158): one visible key returns its value row.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import paged as opaged
from oracle.numerics import f32_to_bf16_bits
from paged_cases import FMT_NAME, make_case, oracle_output, to_numpy_f32

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _decode(case, **kwargs):
    from economize_amd.paged import paged_decode_attention

    cache = case.device_cache()
    table = torch.from_numpy(case.table).cuda()
    lens = torch.tensor(case.lens, dtype=torch.int32).cuda()
    out = paged_decode_attention(case.q.cuda(), cache, table, lens, max(max(case.lens), 1), **kwargs)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    # batch, queries, q heads, kv heads, head dim, lengths, dtype
    (1, 1, 8, 2, 64, [512], torch.float8_e4m3fn),  # the CPU-runnable plumbing shape
    (6, 1, 32, 8, 128, [1, 15, 16, 17, 100, 1000], torch.float8_e4m3fn),
    (3, 1, 32, 8, 128, [300, 64, 1025], torch.bfloat16),
    (2, 1, 16, 4, 128, [700, 33], torch.float8_e5m2),
    (2, 4, 16, 2, 128, [260, 71], torch.float8_e4m3fn),  # verification: 32 rows per KV head, causal
    (2, 8, 64, 8, 128, [200, 129], torch.float8_e4m3fn),  # 64 rows per KV head
    (2, 2, 8, 8, 256, [90, 300], torch.bfloat16),
    (2, 1, 8, 2, 256, [2000, 3333], torch.bfloat16),  # long rows at D = 256
    (2, 1, 8, 2, 256, [2000, 3333], torch.float8_e4m3fn),
    (3, 1, 4, 4, 64, [0, 5, 40], torch.float8_e4m3fn),  # an empty row gives zeros
    (1, 1, 32, 8, 128, [32768], torch.float8_e4m3fn),  # rows cut into many waves' ranges
    (40, 1, 8, 1, 128, [3 + 97 * i for i in range(40)], torch.float8_e4m3fn),  # many short rows per wave
    (5, 2, 8, 2, 64, [300, 0, 0, 17, 1], torch.bfloat16),  # empty rows between others
    (70, 1, 8, 2, 64, [(37 * i) % 700 for i in range(70)], torch.float8_e4m3fn),  # more than 64 batch rows
    (2, 6, 64, 4, 128, [300, 90], torch.float8_e4m3fn),  # 96 rows per KV head: query chunks of 4 + 2
    (2, 12, 16, 2, 64, [500, 40], torch.bfloat16),  # 96 rows per KV head: query chunks of 8 + 4
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}q{c[1]}h{c[2]}k{c[3]}d{c[4]}-{str(c[6])[6:]}" for c in CASES])
def test_decode_matches_the_oracle(case) -> None:
    batch, queries, hq, hkv, d, lens, dtype = case
    c = make_case(batch, queries, hq, hkv, d, lens, dtype, seed=sum(lens) + d)
    got = _decode(c)
    want = oracle_output(c)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)
    for b, n in enumerate(lens):
        if n == 0:
            assert (got[b] == 0).all()


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.float8_e5m2, torch.bfloat16])
def test_slots_past_each_row_may_hold_nan_codes(dtype) -> None:
    """Cache memory a row does not hold (the rest of its last page, unused pages) is never read into the result,
    whatever it holds: the reference's kernels load K/V with a mask (attention/_decode_kernels.py:161-171)."""
    from economize_amd.paged import paged_decode_attention

    lens = [1, 17, 250, 1000, 31]
    c = make_case(5, 1, 16, 4, 128, lens, dtype, seed=5)
    cache = c.device_cache(poison=True)
    table = torch.from_numpy(c.table).cuda()
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    out = paged_decode_attention(c.q.cuda(), cache, table, seq, max(lens)).float().cpu().numpy()
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, oracle_output(c), atol=ATOL, rtol=RTOL)


def test_repeated_calls_reset_the_split_counters() -> None:
    """The merging split resets its row's counter: calls on one workspace keep agreeing with the oracle, for rows
    with one split, several splits and none."""
    from economize_amd.paged import new_workspace, paged_decode_attention, workspace_size

    c = make_case(4, 1, 32, 8, 128, [4000, 20, 0, 2500], torch.float8_e4m3fn, seed=11)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    lens = torch.tensor(c.lens, dtype=torch.int32).cuda()
    ws = new_workspace(workspace_size(4, 1, 32, 8, 128, 4000), "cuda")
    want = oracle_output(c)
    for _ in range(3):
        out = paged_decode_attention(c.q.cuda(), cache, table, lens, 4000, workspace=ws)
        np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    counters = ws[: 4 * 8 * 4].view(torch.int32)
    assert int(counters.abs().sum()) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_page_list_attends_the_selected_pages_and_the_tail(dtype) -> None:
    """Quest's gathered attention (attention/quest.py:239-344) through the page list: the oracle's selection
    (quest.py:73-108) over the decoded keys, then attention over the selected pages and the dense tail
    (quest.py:207-219)."""
    from oracle import quest as oquest

    lens = [2000, 700, 64, 1100]
    c = make_case(4, 1, 16, 4, 128, lens, dtype, seed=21)
    kd, vd = c.decoded()
    done = np.array([(n - 1) // 16 for n in lens])
    max_done = int(done.max())
    pages = 9
    kmin, kmax = oquest.page_bounds(kd, 0, max_done, 16)
    q = to_numpy_f32(c.q).transpose(0, 2, 1, 3)
    index = oquest.select_pages(q, kmin, kmax, done, max_done, pages)
    got = _decode(c, page_list=torch.from_numpy(index).cuda(), done=torch.from_numpy(done.astype(np.int32)).cuda())
    visible = (np.arange(kd.shape[2])[None, :] < np.array(lens)[:, None])[:, None, None, :]  # each row's tokens
    want = oquest.quest_reference(q, kd, vd, visible, 1 / np.sqrt(128), index, done, 16)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


def test_softcap_and_sinks() -> None:
    c = make_case(2, 2, 16, 4, 128, [333, 50], torch.float8_e4m3fn, seed=7)
    sinks = np.random.default_rng(0).standard_normal(16).astype(np.float32)
    got = _decode(c, softcap=5.0, sinks=torch.from_numpy(sinks).cuda(), scale=0.3)
    want = oracle_output(c, scale=0.3, softcap=5.0, sinks=sinks)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_every_fp8_byte_decodes_exactly(dtype) -> None:
    from economize_amd.paged import PagedKVCache, paged_decode_attention

    raw = np.arange(256, dtype=np.uint8)
    table = ofp8.decode_table(FMT_NAME[dtype])
    raw = np.where(np.isfinite(table), raw, 0).astype(np.uint8)
    d = 256
    cache = PagedKVCache.empty(1, 1, d, dtype, "cuda")
    v = np.zeros((1, 1, 16, d), np.uint8)
    v[0, 0, 0] = raw
    kc, vc = opaged.scatter_kv(np.zeros((1, 1, 16, d), np.uint8), v, [16], np.zeros((1, 1), np.int32), 1, 16, 1)
    cache.keys.copy_(torch.from_numpy(kc).view(dtype))
    cache.values.copy_(torch.from_numpy(vc).view(dtype))
    q = torch.zeros(1, 1, 2, d, dtype=torch.bfloat16, device="cuda")
    out = paged_decode_attention(q, cache, torch.zeros(1, 1, dtype=torch.int32, device="cuda"),
                                 torch.ones(1, dtype=torch.int32, device="cuda"), 1)
    want = table[raw]
    got = out[0, 0].float().cpu().numpy()
    assert np.array_equal(got[0], want) and np.array_equal(got[1], want)


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.float8_e5m2, torch.bfloat16])
def test_append_writes_the_oracle_codes(dtype) -> None:
    from economize_amd.paged import PagedKVCache, head_scales, paged_append

    gen = torch.Generator().manual_seed(3)
    lens = [37, 16, 70]
    hkv, d = 4, 128
    k = (torch.randn(3, hkv, 70, d, generator=gen) * 3).to(torch.bfloat16)
    v = torch.randn(3, hkv, 70, d, generator=gen).to(torch.bfloat16)
    k[0, 1, 5, 7] = 1e4  # an outlier sets head 1's key scale
    table, pages = opaged.shuffled_block_table(lens, 16, seed=4)
    kf, vf = to_numpy_f32(k), to_numpy_f32(v)
    mask = np.zeros((3, 1, 70, 1), bool)
    for b, n in enumerate(lens):
        mask[b, :, :n] = True
    scaled = dtype != torch.bfloat16
    if scaled:
        fmt = FMT_NAME[dtype]
        ks_np = ofp8.head_scales(np.where(mask, kf, 0), fmt)
        vs_np = ofp8.head_scales(np.where(mask, vf, 0), fmt)
        ks = head_scales(torch.where(torch.from_numpy(mask), k, 0).cuda(), dtype)
        vs = head_scales(torch.where(torch.from_numpy(mask), v, 0).cuda(), dtype)
        assert np.array_equal(ks.cpu().numpy(), ks_np) and np.array_equal(vs.cpu().numpy(), vs_np)
        want_k = ofp8.fp8_encode(kf, fmt, ks_np.reshape(1, -1, 1, 1))
        want_v = ofp8.fp8_encode(vf, fmt, vs_np.reshape(1, -1, 1, 1))
        element = 1
    else:
        ks = vs = None
        want_k, want_v = f32_to_bf16_bits(kf), f32_to_bf16_bits(vf)
        element = 2
    cache = PagedKVCache.empty(pages, hkv, d, dtype, "cuda", ks, vs)
    for b, n in enumerate(lens):
        # appended in two passes: a prompt, then the rest one token at a time in a batch with a padding slot
        cut = n // 2
        slots = torch.from_numpy(opaged.slot_mapping(table, b, 0, cut, 16)).cuda()
        paged_append(cache, k[b, :, :cut].transpose(0, 1).cuda(), v[b, :, :cut].transpose(0, 1).cuda(), slots)
        for t in range(cut, n):
            slot = opaged.slot_mapping(table, b, t, 1, 16)
            slots = torch.tensor([slot[0], -1], dtype=torch.int32).cuda()
            kk = k[b, :, t: t + 1].transpose(0, 1).repeat(2, 1, 1).cuda()
            vv = v[b, :, t: t + 1].transpose(0, 1).repeat(2, 1, 1).cuda()
            paged_append(cache, kk, vv, slots)
    torch.cuda.synchronize()
    raw = torch.int16 if element == 2 else torch.uint8
    got_k = cache.keys.view(raw).cpu().numpy()
    got_v = cache.values.view(raw).cpu().numpy()
    if element == 2:
        got_k, got_v = got_k.view(np.uint16), got_v.view(np.uint16)
    want_kc, want_vc = opaged.scatter_kv(want_k, want_v, lens, table, pages, 16, element)
    assert np.array_equal(got_k, want_kc) and np.array_equal(got_v, want_vc)


F16_CASES = [
    # batch, queries, q heads, kv heads, head dim, lengths, dtype
    (1, 1, 8, 2, 64, [512], torch.float8_e4m3fn),
    (6, 1, 32, 8, 128, [1, 15, 16, 17, 100, 1000], torch.float8_e4m3fn),
    (2, 1, 16, 4, 128, [700, 33], torch.float8_e5m2),
    (2, 4, 16, 2, 128, [260, 71], torch.float8_e4m3fn),  # verification: 32 rows per KV head, causal
    (2, 8, 64, 8, 128, [200, 129], torch.float8_e4m3fn),  # 64 rows per KV head
    (2, 1, 8, 2, 256, [2000, 3333], torch.float8_e4m3fn),
    (3, 1, 4, 4, 64, [0, 5, 40], torch.float8_e5m2),  # an empty row gives zeros
    (2, 6, 64, 4, 128, [300, 90], torch.float8_e4m3fn),  # query chunks
]


@pytest.mark.parametrize("case", F16_CASES,
                         ids=[f"b{c[0]}q{c[1]}h{c[2]}k{c[3]}d{c[4]}-{str(c[6])[6:]}" for c in F16_CASES])
def test_fp16_queries_over_an_fp8_cache(case) -> None:
    """A model in fp16 with its cache in fp8: fp16 queries (the keys converted to fp16 exactly for the fp16 MFMA) and
    an fp16 output, within the same tolerance of the fp32 definition; soft cap and sinks on one case."""
    from economize_amd.paged import paged_decode_attention

    batch, queries, hq, hkv, d, lens, dtype = case
    c = make_case(batch, queries, hq, hkv, d, lens, dtype, seed=sum(lens) + d + 1)
    gen = torch.Generator().manual_seed(len(lens) + d)
    c.q = (torch.randn(c.q.shape, generator=gen) * 1.5).to(torch.float16)
    extra = {}
    if hq == 16 and d == 128 and queries == 1:
        extra = {"softcap": 30.0, "sinks": torch.randn(hq, generator=gen)}
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    seq = torch.tensor(c.lens, dtype=torch.int32).cuda()
    out = paged_decode_attention(c.q.cuda(), cache, table, seq, max(max(c.lens), 1), softcap=extra.get("softcap"),
                                 sinks=None if "sinks" not in extra else extra["sinks"].cuda())
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    got = out.float().cpu().numpy()
    want = oracle_output(c, softcap=extra.get("softcap"),
                         sinks=None if "sinks" not in extra else extra["sinks"].numpy())
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)
    for b, n in enumerate(lens):
        if n == 0:
            assert (got[b] == 0).all()


def test_bad_arguments_raise_before_launch() -> None:
    from economize_amd.errors import ConfigError
    from economize_amd.paged import PagedKVCache, paged_decode_attention

    cache = PagedKVCache.empty(2, 2, 128, torch.float8_e4m3fn, "cuda")
    q = torch.zeros(1, 1, 3, 128, dtype=torch.bfloat16, device="cuda")  # 3 query heads over 2 KV heads
    table = torch.zeros(1, 2, dtype=torch.int32, device="cuda")
    lens = torch.ones(1, dtype=torch.int32, device="cuda")
    with pytest.raises(ConfigError):
        paged_decode_attention(q, cache, table, lens, 1)
    with pytest.raises(ConfigError):
        paged_decode_attention(torch.zeros(1, 1, 4, 128, device="cuda"), cache, table, lens, 1)  # fp32 query
    bf16_cache = PagedKVCache.empty(2, 2, 128, torch.bfloat16, "cuda")
    q16 = torch.zeros(1, 1, 4, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(ConfigError, match="fp16 queries"):
        paged_decode_attention(q16, bf16_cache, table, lens, 1)  # fp16 queries read an fp8 cache only
    with pytest.raises(ConfigError, match="fp16 queries"):
        paged_decode_attention(q16, cache, table, lens, 1, page_list=torch.zeros(1, 2, 1, dtype=torch.int32,
                                                                                 device="cuda"),
                               done=torch.zeros(1, dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("dtype,kind,queries,hq", [(torch.float8_e4m3fn, "broadcast", 1, 32),
                                                   (torch.bfloat16, "per_head", 2, 16),
                                                   (torch.float8_e4m3fn, "per_head", 8, 64),
                                                   (torch.float8_e4m3fn, "per_head", 12, 64)])  # query chunks
def test_decode_with_a_mask(dtype, kind, queries, hq) -> None:
    """An attention mask (key t = token t of the row; bool, broadcast or per head) hides keys on top of the causal
    limit, as the reference's decode_attention takes a mask (attention/decode.py:252-300)."""
    from oracle.attention import reference_attention

    lens = [700, 90, 1500]
    c = make_case(3, queries, hq, 8, 128, lens, dtype, seed=77 + queries)
    rng = np.random.default_rng(78)
    smax = max(lens)
    shape = (1, 1, 1, smax + 5) if kind == "broadcast" else (3, hq, queries, smax)
    mask = rng.random(shape) < 0.6
    got = _decode(c, mask=torch.from_numpy(mask).cuda())
    kd, vd = c.decoded()
    causal = np.zeros((3, 1, queries, smax), bool)
    for b, n in enumerate(lens):
        for qi in range(queries):
            causal[b, 0, qi, : n - queries + qi + 1] = True
    q = to_numpy_f32(c.q).transpose(0, 2, 1, 3)
    want = reference_attention(q, kd, vd, causal & mask[..., :smax], 1 / np.sqrt(128))
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


def test_mask_bits_pack_the_bool_mask() -> None:
    """eco_mask_bits: bit t % 32 of word t / 32 is mask[..., t], words past the keys hold zeros."""
    from economize_amd.paged import packed_mask

    rng = np.random.default_rng(5)
    mask = rng.random((2, 3, 4, 77)) < 0.5
    bits, strides, words = packed_mask(torch.from_numpy(mask).cuda(), 2, 3, 4)
    assert words == 3 and strides == (3 * 4 * 3, 4 * 3, 3)
    got = bits.cpu().numpy().view(np.uint32)
    want = np.zeros((2, 3, 4, 3), np.uint32)
    for t in range(77):
        want[..., t // 32] |= mask[..., t].astype(np.uint32) << np.uint32(t % 32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype,out", [(torch.float8_e4m3fn, torch.bfloat16), (torch.float8_e5m2, torch.float32),
                                       (torch.bfloat16, torch.float16)])
def test_gather_gives_the_dense_view(dtype, out) -> None:
    """eco_paged_gather: the stored K/V of every row's tokens, fp8 decoded exactly times the head scales, in the
    output dtype; 0 past a row's pages."""
    from economize_amd.paged import paged_gather

    lens = [300, 17, 0, 129]
    c = make_case(4, 1, 8, 2, 64, lens, dtype, seed=61)
    cache = c.device_cache()
    keys = max(lens)
    k, v = paged_gather(cache, torch.from_numpy(c.table).cuda(), keys, out)
    assert k.dtype == out and k.shape == (4, 2, keys, 64)
    kd, vd = c.decoded()
    held = (np.arange(keys)[None, :] < np.array(lens)[:, None])[:, None, :, None]
    want_k = torch.from_numpy(np.where(held, kd[:, :, :keys], 0)).to(out).float().numpy()
    want_v = torch.from_numpy(np.where(held, vd[:, :, :keys], 0)).to(out).float().numpy()
    got_k, got_v = k.float().cpu().numpy(), v.float().cpu().numpy()
    assert np.array_equal(np.where(held, got_k, 0), want_k) and np.array_equal(np.where(held, got_v, 0), want_v)


def sweep_case(i: int):
    """Randomized paged decode case ``i``: cache dtype, head dim, GQA, query count (up to 96 rows per KV head, so
    query chunks), batch and lengths (empty, shorter than a tile, long), and whether a per-query mask applies, drawn
    from a seeded generator on the CPU."""
    rng = np.random.default_rng(50_000 + i)
    dtype = [torch.float8_e4m3fn, torch.float8_e5m2, torch.bfloat16][int(rng.integers(0, 3))]
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    groups = int(rng.choice([1, 2, 4, 8, 16]))
    queries = int(rng.integers(1, 7))
    batch = int(rng.integers(1, 6))
    lens = []
    for _ in range(batch):
        kind = rng.random()
        if kind < 0.1:
            lens.append(0)
        elif kind < 0.3:
            lens.append(int(rng.integers(max(queries, 1), 80)))
        else:
            lens.append(int(rng.integers(80, 2500)))
    return batch, queries, groups * hkv, hkv, d, lens, dtype, bool(rng.random() < 0.25), 60_000 + i


SWEEP = [sweep_case(i) for i in range(200)]


@pytest.mark.parametrize("case", SWEEP, ids=[f"{i}-b{c[0]}q{c[1]}h{c[2]}k{c[3]}d{c[4]}-{str(c[6])[6:]}"
                                             f"{'-mask' if c[7] else ''}" for i, c in enumerate(SWEEP)])
def test_randomized_sweep(case) -> None:
    from oracle.attention import reference_attention

    batch, queries, hq, hkv, d, lens, dtype, masked, seed = case
    if max(lens) == 0:
        lens = lens[:-1] + [1]
    c = make_case(batch, queries, hq, hkv, d, lens, dtype, seed=seed)
    mask = None
    if masked:
        mask = np.random.default_rng(seed + 1).random((batch, hq, queries, max(lens))) < 0.7
    got = _decode(c, mask=None if mask is None else torch.from_numpy(mask).cuda())
    if mask is None:
        want = oracle_output(c)
    else:
        kd, vd = c.decoded()
        smax = max(lens)
        causal = np.zeros((batch, 1, queries, smax), bool)
        for b, n in enumerate(lens):
            for qi in range(queries):
                causal[b, 0, qi, : max(n - queries + qi + 1, 0)] = True
        q = to_numpy_f32(c.q).transpose(0, 2, 1, 3)
        want = reference_attention(q, kd, vd, causal & mask, 1 / np.sqrt(d))
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)
