"""Parity of the KIVI kernels with the oracle on the GPU.

* quantize-and-append: the page blocks (codes, fp16 scales and zero points) bit-exact against the oracle's
  restatement of the reference's ``quantize`` (techniques/kv_quant/kivi.py:121-140) laid out in the paged format
  (oracle/kivi_paged.py), for prompts and for the decode-time schedule (kivi.py:230-243) run step by step;
* decode attention within atol 2e-3 / rtol 1e-2 of the fp32 definition (attention/decode.py:66-103) over the values
  the reference's ``dequantize`` gives (attention/kivi.py:56-76) and the bf16 residual, for 2- and 4-bit codes,
  outlier key channels, GQA, causal verification queries (64 rows per KV head), soft cap and sinks, and caches whose
  unused slots hold NaN.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import kivi_paged as okp
from oracle import paged as opaged
from oracle.attention import reference_attention
from oracle.numerics import bf16_bits_to_f32

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
R, HEADROOM = 128, 256
W = R + HEADROOM


@dataclass
class KiviCase:
    q: torch.Tensor  # [B, Q, Hq, D] bf16 (CPU)
    k: torch.Tensor  # [B, Hkv, S, D] bf16 (CPU)
    v: torch.Tensor
    lens: list[int]
    queries: int
    bits: int
    table: np.ndarray
    pages: int
    kq: np.ndarray
    vq: np.ndarray


def make_case(batch, queries, q_heads, kv_heads, head_dim, lens, bits, seed) -> KiviCase:
    gen = torch.Generator().manual_seed(seed)
    smax = max(lens)
    q = torch.randn(batch, queries, q_heads, head_dim, generator=gen).to(torch.bfloat16)
    k = torch.randn(batch, kv_heads, smax, head_dim, generator=gen)
    v = torch.randn(batch, kv_heads, smax, head_dim, generator=gen)
    outliers = torch.randperm(head_dim, generator=gen)[:4 * head_dim // 128 or 1]
    k[..., outliers] *= 10.0  # outlier key channels, as in KIVI's analysis
    table, pages = opaged.shuffled_block_table(lens, okp.PAGE, seed=seed + 1)
    committed = np.array([n - queries for n in lens])
    kq = (committed // R) * R
    vq = np.maximum(committed - R, 0)
    return KiviCase(q, k.to(torch.bfloat16), v.to(torch.bfloat16), list(lens), queries, bits, table, pages,
                    kq.astype(np.int32), vq.astype(np.int32))


def oracle_blocks(c: KiviCase, head_dim: int, rows=None) -> np.ndarray:
    kv_heads = c.k.shape[1]
    size = okp.block_layout(head_dim, c.bits, 32)["size"]
    blocks = np.zeros((c.pages, kv_heads, size), np.uint8)
    kf, vf = c.k.float().numpy(), c.v.float().numpy()
    for b in (range(len(c.lens)) if rows is None else rows):
        okp.write_keys(blocks, kf, b, 0, int(c.kq[b]), c.table, c.bits, 32)
        okp.write_values(blocks, vf, b, 0, int(c.vq[b]), c.table, c.bits, 32)
    return blocks


def device_cache(c: KiviCase, poison: bool = False):
    """The GPU cache after a prompt of every row's tokens: codes below kq / vq, the last W tokens in the rings."""
    from economize_amd.kivi import PagedKIVICache, kivi_append, kivi_quantize

    batch, kv_heads, smax, head_dim = c.k.shape
    cache = PagedKIVICache.empty(c.pages, batch, kv_heads, head_dim, c.bits, "cuda", residual=R, headroom=HEADROOM)
    if poison:  # never-written memory: NaN scales, zero points and ring entries
        cache.blocks.fill_(0xFF)
        cache.k_ring.fill_(float("nan"))
        cache.v_ring.fill_(float("nan"))
    table = torch.from_numpy(c.table).cuda()
    zeros = torch.zeros(batch, dtype=torch.int32, device="cuda")
    kivi_quantize(cache, table, c.k.cuda(), "k", zeros, torch.from_numpy(c.kq).cuda(), int(c.kq.max()))
    kivi_quantize(cache, table, c.v.cuda(), "v", zeros, torch.from_numpy(c.vq).cuda(), int(c.vq.max()))
    rows, pos = [], []
    for b, n in enumerate(c.lens):
        for t in range(max(0, n - W), n):
            rows.append(b)
            pos.append(t)
    rows_t = torch.tensor(rows, dtype=torch.int32)
    pos_t = torch.tensor(pos, dtype=torch.int32)
    kk = c.k[rows_t.long(), :, pos_t.long()]  # [T, Hkv, D]
    vv = c.v[rows_t.long(), :, pos_t.long()]
    kivi_append(cache, kk.cuda(), vv.cuda(), rows_t.cuda(), pos_t.cuda())
    cache.keys_quantized.copy_(torch.from_numpy(c.kq))
    cache.values_quantized.copy_(torch.from_numpy(c.vq))
    return cache, table


def oracle_output(c: KiviCase, scale=None, softcap=None, sinks=None, rows=None, mask=None) -> np.ndarray:
    """The fp32 attention (decode.py:66-103) over the keys and values the reference's ``dequantize`` gives from the
    oracle's pages, and the bf16 residual; ``[B, Q, Hq, D]``, only the batch ``rows`` given (all by default). An
    extra boolean ``mask`` ``[B or 1, Hq or 1, Q or 1, >= S]`` hides keys on top of the causal limit."""
    batch, kv_heads, smax, head_dim = c.k.shape
    rows = list(range(batch)) if rows is None else list(rows)
    blocks = oracle_blocks(c, head_dim, rows)
    kf, vf = c.k.float().numpy(), c.v.float().numpy()
    k_ring = np.zeros((batch, kv_heads, W, head_dim), np.float32)
    v_ring = np.zeros((batch, kv_heads, head_dim, W), np.float32)
    for b in rows:
        n = c.lens[b]
        slots = np.arange(max(0, n - W), n)
        k_ring[b][:, slots % W] = kf[b][:, slots]
        v_ring[b][:, :, slots % W] = vf[b][:, slots].transpose(0, 2, 1)
    keys, values = okp.dense_view(blocks, c.table, k_ring, v_ring, c.lens, c.kq, c.vq, c.bits, 32, rows=rows)
    q = c.q.float().numpy().transpose(0, 2, 1, 3)
    scale = 1 / np.sqrt(head_dim) if scale is None else scale
    out = np.zeros((batch, c.queries, q.shape[1], head_dim), np.float32)
    for b in rows:
        n = c.lens[b]
        causal = np.zeros((1, 1, c.queries, smax), bool)
        for qi in range(c.queries):
            causal[0, 0, qi, : n - c.queries + qi + 1] = True
        if mask is not None:
            causal = causal & mask[b if mask.shape[0] > 1 else 0][None, ..., :smax]
        out[b] = reference_attention(q[b:b + 1], keys[b:b + 1], values[b:b + 1], causal, scale, softcap=softcap,
                                     sinks=sinks)[0]
    return out


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_prompt_quantization_matches_the_oracle(bits, head_dim) -> None:
    c = make_case(3, 1, 8, 2, head_dim, [700, 300, 1025], bits, seed=bits + head_dim)
    cache, _ = device_cache(c)
    torch.cuda.synchronize()
    got = cache.blocks.cpu().numpy()
    want = oracle_blocks(c, head_dim)
    assert np.array_equal(got, want)
    assert int(cache.overflow.item()) == 0


def test_scales_beyond_the_fp16_range_are_refused() -> None:
    """The reference's test_scales_beyond_the_fp16_range_are_refused (tests/techniques/test_kv_kivi_packed.py:
    158-164): keys 1e5 times larger quantize to scales and zero points beyond fp16, which the packed pages cannot
    hold; the device flag turns into a ConfigError at the next check, which clears it."""
    import dataclasses

    from economize_amd.errors import ConfigError

    c = make_case(1, 1, 8, 2, 64, [300], 2, seed=5)
    c = dataclasses.replace(c, k=(c.k.float() * 1e5).to(torch.bfloat16))
    cache, _ = device_cache(c)
    with pytest.raises(ConfigError, match="fp16"):
        cache.check_flags()
    cache.check_flags()


def test_decode_time_schedule_matches_one_shot_quantization() -> None:
    """Tokens appended one at a time with the schedule run after every step (kivi_commit) leave the same pages and
    counts as quantizing the final prefixes at once."""
    from economize_amd.kivi import PagedKIVICache, kivi_append, kivi_commit

    bits, head_dim, kv_heads = 4, 128, 2
    lens = [200, 131]
    c = make_case(2, 1, 8, kv_heads, head_dim, lens, bits, seed=5)
    cache = PagedKIVICache.empty(c.pages, 2, kv_heads, head_dim, bits, "cuda", residual=R, headroom=HEADROOM)
    table = torch.from_numpy(c.table).cuda()
    for t in range(max(lens)):
        rows = [b for b, n in enumerate(lens) if t < n]
        kk = c.k[rows, :, t]
        vv = c.v[rows, :, t]
        kivi_append(cache, kk.cuda(), vv.cuda(), torch.tensor(rows, dtype=torch.int32).cuda(),
                    torch.full((len(rows),), t, dtype=torch.int32).cuda())
        committed = torch.tensor([min(t + 1, n) for n in lens], dtype=torch.int32).cuda()
        kivi_commit(cache, table, committed, 1)
    torch.cuda.synchronize()
    c.kq = np.array([(n // R) * R for n in lens], np.int32)
    c.vq = np.array([max(n - R, 0) for n in lens], np.int32)
    assert np.array_equal(cache.keys_quantized.cpu().numpy(), c.kq)
    assert np.array_equal(cache.values_quantized.cpu().numpy(), c.vq)
    assert np.array_equal(cache.blocks.cpu().numpy(), oracle_blocks(c, head_dim))


CASES = [
    # batch, queries, q heads, kv heads, head dim, lengths, bits
    (3, 1, 32, 8, 128, [1000, 333, 2050], 2),
    (3, 1, 32, 8, 128, [1000, 333, 2050], 4),
    (2, 1, 8, 2, 64, [700, 129], 2),
    (2, 1, 16, 4, 64, [90, 520], 4),
    (2, 8, 64, 8, 128, [1500, 1100], 4),  # verification: 8 draft tokens x GQA 8 = 64 rows per KV head
    (2, 5, 64, 8, 64, [900, 300], 2),  # 40 rows: the last 16-row block of the workgroup holds none
    (1, 8, 64, 8, 128, [6000], 2),  # 64 rows of one long row cut between workgroups
    (3, 4, 128, 8, 64, [513, 2000, 64], 4),  # GQA 16 x 4 queries = 64 rows at head dim 64
    (4, 2, 16, 2, 128, [40, 1, 160, 385], 2),  # rows shorter than the residual: no codes at all
    (1, 1, 32, 8, 128, [8192], 2),  # one long row cut into many waves' ranges
    (2, 12, 64, 8, 128, [1300, 400], 4),  # 96 rows per KV head: query chunks of 8 (64 rows) + 4 (32 rows)
    (2, 5, 128, 4, 64, [700, 150], 2),  # 32 query heads per KV head x 5 queries: chunks of 2, 2, 1
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}q{c[1]}h{c[2]}k{c[3]}d{c[4]}-int{c[6]}" for c in CASES])
def test_decode_matches_the_oracle(case) -> None:
    from economize_amd.kivi import kivi_decode_attention

    batch, queries, hq, hkv, d, lens, bits = case
    c = make_case(batch, queries, hq, hkv, d, lens, bits, seed=sum(lens) + bits)
    cache, table = device_cache(c)
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, max(lens)).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle_output(c), atol=ATOL, rtol=RTOL)


# Cases where a value product that does not round every dequantized value to bf16 (as the reference does before its
# P.V dot) lies beyond atol / rtol of the reference: the kernel must give the reference's values.
ROUNDING_CASES = [
    (3, 4, 64, 8, 128, [1388, 201, 2308], 4, 1001),
    (4, 8, 8, 2, 64, [402, 1737, 50, 1541], 4, 1017),
]


@pytest.mark.parametrize("case", ROUNDING_CASES, ids=[f"b{c[0]}q{c[1]}h{c[2]}k{c[3]}d{c[4]}-int{c[6]}"
                                                      for c in ROUNDING_CASES])
def test_values_are_rounded_as_the_reference_rounds_them(case) -> None:
    from economize_amd.kivi import kivi_decode_attention

    batch, queries, hq, hkv, d, lens, bits, seed = case
    c = make_case(batch, queries, hq, hkv, d, lens, bits, seed=seed)
    cache, table = device_cache(c)
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, max(lens)).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle_output(c), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("queries,hq", [(1, 32), (8, 64)])
def test_large_values(bits, queries, hq) -> None:
    """Values 1000 times larger (32-channel ranges of about 6000, value scales up to 2000 at int2): every product of
    the value path is fp32, so nothing overflows, and the output stays within tolerance."""
    import dataclasses

    from economize_amd.kivi import kivi_decode_attention

    c = make_case(2, queries, hq, 8, 128, [1500, 700], bits, seed=31 + bits)
    c = dataclasses.replace(c, v=(c.v.float() * 1000).to(torch.bfloat16))
    cache, table = device_cache(c)
    cache.check_flags()  # the scales fit fp16
    seq = torch.tensor(c.lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, max(c.lens)).float().cpu().numpy()
    assert np.isfinite(got).all()
    assert np.abs(got).max() > 100
    np.testing.assert_allclose(got, oracle_output(c), atol=ATOL, rtol=RTOL)


def sweep_case(i: int):
    """Randomized KIVI decode case ``i``: head dim, bits, GQA, query count, batch and lengths (some shorter than the
    residual, some holding only the queries), drawn from a seeded generator on the CPU."""
    rng = np.random.default_rng(20_000 + i)
    d = int(rng.choice([64, 128]))
    bits = int(rng.choice([2, 4]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    groups = int(rng.choice([1, 2, 4, 8, 16]))
    queries = int(rng.integers(1, 9))
    while groups * queries > 64:
        queries -= 1
    batch = int(rng.integers(1, 5))
    lens = []
    for _ in range(batch):
        kind = rng.random()
        if kind < 0.15:
            lens.append(queries)
        elif kind < 0.35:
            lens.append(int(rng.integers(queries, 200)))
        else:
            lens.append(int(rng.integers(max(queries, 200), 2600)))
    return batch, queries, groups * hkv, hkv, d, lens, bits, 40_000 + i


SWEEP = [sweep_case(i) for i in range(200)]


@pytest.mark.parametrize("case", SWEEP, ids=[f"{i}-b{c[0]}q{c[1]}h{c[2]}k{c[3]}d{c[4]}-int{c[6]}"
                                             for i, c in enumerate(SWEEP)])
def test_randomized_sweep(case) -> None:
    from economize_amd.kivi import kivi_decode_attention

    batch, queries, hq, hkv, d, lens, bits, seed = case
    c = make_case(batch, queries, hq, hkv, d, lens, bits, seed=seed)
    cache, table = device_cache(c)
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, max(lens)).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle_output(c), atol=ATOL, rtol=RTOL)


def test_unused_slots_may_hold_nan() -> None:
    from economize_amd.kivi import kivi_decode_attention

    c = make_case(3, 1, 16, 4, 128, [1000, 77, 450], 4, seed=17)
    cache, table = device_cache(c, poison=True)
    seq = torch.tensor(c.lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, max(c.lens)).float().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, oracle_output(c), atol=ATOL, rtol=RTOL)


def test_softcap_and_sinks() -> None:
    from economize_amd.kivi import kivi_decode_attention

    c = make_case(2, 2, 16, 4, 128, [600, 333], 2, seed=23)
    cache, table = device_cache(c)
    sinks = np.random.default_rng(1).standard_normal(16).astype(np.float32)
    seq = torch.tensor(c.lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, max(c.lens), scale=0.2, softcap=4.0,
                                sinks=torch.from_numpy(sinks).cuda()).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle_output(c, scale=0.2, softcap=4.0, sinks=sinks), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("kind,queries,hq", [("broadcast", 1, 32), ("per_head", 2, 16), ("per_head", 8, 64),
                                             ("per_head", 12, 64)])
def test_decode_with_a_mask(kind, queries, hq) -> None:
    """An attention mask (key t = token t of the row) hides keys on top of the causal limit, as the reference's
    kernels take a mask (attention/_kivi_kernels.py:176-183); with 64 query rows the verification kernel runs, with
    96 two query chunks."""
    from economize_amd.kivi import kivi_decode_attention

    lens = [1100, 70, 600]
    c = make_case(3, queries, hq, 8, 128, lens, 4, seed=81 + queries)
    cache, table = device_cache(c)
    rng = np.random.default_rng(82)
    smax = max(lens)
    shape = (1, 1, 1, smax + 7) if kind == "broadcast" else (3, hq, queries, smax)
    mask = rng.random(shape) < 0.6
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    got = kivi_decode_attention(c.q.cuda(), cache, table, seq, smax,
                                mask=torch.from_numpy(mask).cuda()).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle_output(c, mask=mask), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("bits", [2, 4])
def test_gather_gives_the_dense_view(bits) -> None:
    """eco_kivi_gather: keys below kq and values below vq dequantized as the reference's dequantize (bf16), the
    others from the rings: the oracle's dense view of the same pages and rings, bit for bit."""
    from economize_amd.kivi import kivi_gather

    c = make_case(3, 1, 8, 2, 128, [700, 77, 450], bits, seed=90 + bits)
    cache, table = device_cache(c)
    k, v = kivi_gather(cache, table, max(c.lens))
    blocks = oracle_blocks(c, 128)
    batch, kv_heads, smax, head_dim = c.k.shape
    kf, vf = c.k.float().numpy(), c.v.float().numpy()
    k_ring = np.zeros((batch, kv_heads, W, head_dim), np.float32)
    v_ring = np.zeros((batch, kv_heads, head_dim, W), np.float32)
    for b, n in enumerate(c.lens):
        for t in range(max(0, n - W), n):
            k_ring[b, :, t % W] = kf[b, :, t]
            v_ring[b, :, :, t % W] = vf[b, :, t]
    want_k, want_v = okp.dense_view(blocks, c.table, k_ring, v_ring, c.lens, c.kq, c.vq, bits, 32)
    for b, n in enumerate(c.lens):
        assert np.array_equal(k[b, :, :n].float().cpu().numpy(), want_k[b, :, :n])
        assert np.array_equal(v[b, :, :n].float().cpu().numpy(), want_v[b, :, :n])
