"""KIVI on vLLM's cell layout on the GPU (``eco_kivi_cells_quantize``, the reference's quantize_committed,
backends/vllm/kivi/kernels.py:94-207) against the oracle's write_cells (layout.py:222-256), byte for byte: requests
of ragged lengths in shuffled pages, a prefilling request and one without queries left untouched, bf16 / fp16 /
fp32 entries, 2 / 4 / 8 bits, groups of 16 and 32, a second pass that quantizes only what crossed the residual since
the first, a group whose scale overflows fp16, and clear_flags."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import vllm_cells as oc

pytestmark = pytest.mark.gpu

NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def setup(dtype, bits, group, head, page, lens, heads=2, seed=0, scale_up=None):
    """A cache whose cells hold every request's dense K/V (flags 0), the requests' full-precision K/V, the table."""
    from economize_amd.vllm_kivi import cell_layout

    layout = cell_layout(head, dtype, bits, group)
    es = layout.element_size
    per_req = max(-(-n // page) for n in lens) + 1
    pages = len(lens) * per_req + 3
    gen = torch.Generator().manual_seed(seed)
    table = torch.randperm(pages, generator=gen)[: len(lens) * per_req].view(len(lens), per_req).to(torch.int32)
    cache = torch.zeros(pages, heads, page, layout.size // es, dtype=dtype)
    u8 = cache.view(torch.uint8)
    states = []
    for b, n in enumerate(lens):
        k = (torch.randn(heads, n, head, generator=gen) * 2).to(dtype)
        v = (torch.randn(heads, n, head, generator=gen) * 2).to(dtype)
        if scale_up is not None:
            k[:, scale_up] *= 1e6
        states.append((k, v))
        for t in range(n):
            cell = u8[table[b, t // page], :, t % page]
            cell[:, : layout.off_v] = k[:, t].contiguous().view(torch.uint8)
            cell[:, layout.off_v: layout.off_vs] = v[:, t].contiguous().view(torch.uint8)
    return layout, cache, table, states


def expected(layout, cache, table, states, bounds, dtype, page):
    """The cache after write_cells(k, v, kq_b, vq_b) of every request."""
    want = cache.view(torch.uint8).clone().numpy()
    for b, ((k, v), (kq, vq)) in enumerate(zip(states, bounds)):
        if kq == 0 and vq == 0:
            continue
        cells = oc.write_cells(k.float().numpy(), v.float().numpy(), kq, vq, layout, NAMES[dtype])
        for t in range(k.shape[1]):
            want[table[b, t // page], :, t % page, : layout.size] = cells[:, t]
    return want


def run(cache, layout, residual, table, qlens, lens, prefilling):
    from economize_amd.vllm_kivi import quantize_committed

    qsl = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32).cuda()
    quantize_committed(cache, layout, residual, table.cuda(), qsl, torch.tensor(lens, dtype=torch.int32).cuda(),
                       torch.tensor(prefilling, dtype=torch.int32).cuda())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits,group,head,page", [(2, 32, 128, 32), (4, 16, 64, 32), (8, 32, 64, 64),
                                                  (2, 16, 16, 16)])
def test_quantized_cells_match_write_cells(dtype, bits, group, head, page) -> None:
    residual = 2 * group
    lens = [9 * group + 7, 3 * group + 1, 5 * group, 4 * group + 3, 2 * group]
    qlens = [1, 4, 1, 0, 1]            # request 3 has no query this pass
    prefilling = [0, 0, 1, 0, 0]       # request 2 is still prefilling
    layout, cache, table, states = setup(dtype, bits, group, head, page, lens, seed=bits + group + head)
    gpu = cache.cuda()
    run(gpu, layout, residual, table, qlens, lens, prefilling)
    bounds = []
    for n, q, pre in zip(lens, qlens, prefilling):
        c = n - q
        bounds.append((0, 0) if pre or q == 0 or c <= 0 else ((c // residual) * residual, max(0, c - residual)))
    want = expected(layout, cache, table, states, bounds, dtype, page)
    got = gpu.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, want)


def test_a_second_pass_quantizes_what_crossed_the_residual() -> None:
    dtype, bits, group, head, page = torch.bfloat16, 2, 32, 128, 32
    residual = 64
    lens = [300, 200]
    layout, cache, table, states = setup(dtype, bits, group, head, page, lens, seed=11)
    gpu = cache.cuda()
    run(gpu, layout, residual, table, [1, 1], [230, 150], [0, 0])    # the first pass saw 229 and 149 tokens
    run(gpu, layout, residual, table, [1, 1], [300, 200], [0, 0])    # then 299 and 199
    want = expected(layout, cache, table, states, [(256, 235), (192, 135)], dtype, page)
    # only the cells of the first 300 / 200 tokens exist; later slots of the pages stay zero on both sides
    assert np.array_equal(gpu.view(torch.uint8).cpu().numpy(), want)


def test_an_overflowing_key_group_is_flagged() -> None:
    dtype, bits, group, head, page = torch.float32, 2, 32, 64, 32
    layout, cache, table, states = setup(dtype, bits, group, head, page, [100], heads=1, seed=4, scale_up=slice(0, 32))
    gpu = cache.cuda()
    run(gpu, layout, 32, table, [1], [100], [0])
    want = expected(layout, cache, table, states, [(96, 67)], dtype, page)
    got = gpu.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, want)
    first_page = int(table[0, 0])
    assert (got[first_page, 0, :, layout.off_flag] == oc.FLAG_OVERFLOW).all()


def test_clear_flags() -> None:
    from economize_amd.vllm_kivi import clear_flags

    dtype, bits, group, head, page = torch.bfloat16, 4, 16, 64, 32
    layout, cache, table, _ = setup(dtype, bits, group, head, page, [80], seed=2)
    gpu = cache.cuda()
    run(gpu, layout, 16, table, [1], [80], [0])
    slots = torch.tensor([int(table[0, 0]) * page + 3, -1, int(table[0, 1]) * page + 10], dtype=torch.int32)
    clear_flags(gpu, slots.cuda(), layout)
    u8 = gpu.view(torch.uint8).cpu()
    for slot in (int(slots[0]), int(slots[2])):
        assert (u8[slot // page, :, slot % page, layout.off_flag: layout.off_flag + 2] == 0).all()
    assert (u8[int(table[0, 0]), :, 4, layout.off_flag] == 1).all()


def gathered_cells(cache_u8: np.ndarray, table, b: int, n: int, page: int, layout) -> np.ndarray:
    """uint8 [H, n, cell] of request b's first n tokens."""
    return np.stack([cache_u8[int(table[b, t // page]), :, t % page, : layout.size] for t in range(n)], axis=1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits,group,head,q_heads,page", [(2, 32, 128, 8, 32), (4, 16, 64, 4, 32), (4, 16, 64, 4, 16)])
def test_attention_over_the_cells_matches_the_oracle(dtype, bits, group, head, q_heads, page) -> None:
    """vLLM's varlen queries (1, 4, 0 and 3 of them, ragged lengths) attend causally over their request's cells
    after quantize_committed; the oracle reads the cells back (read_cells) and applies the fp32 definition. Pages of
    16 tokens put a 32-key tile's two halves in different pages."""
    from economize_amd.vllm_kivi import paged_kivi_attention
    from oracle.attention import reference_attention

    residual = 2 * group
    lens = [9 * group + 7, 4 * group + 1, 6 * group, 3 * group + 3]
    qlens = [1, 4, 0, 3]
    layout, cache, table, _ = setup(dtype, bits, group, head, page, lens, seed=bits + head)
    gpu = cache.cuda()
    run(gpu, layout, residual, table, qlens, lens, [0, 0, 0, 0])
    gen = torch.Generator().manual_seed(9)
    query = torch.randn(sum(qlens), q_heads, head, generator=gen).to(dtype)
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32)
    sinks = torch.randn(q_heads, generator=gen) if dtype == torch.bfloat16 else None
    out = paged_kivi_attention(query.cuda(), gpu, layout, table.cuda(), qsl.cuda(),
                               torch.tensor(lens, dtype=torch.int32).cuda(), max(qlens), max(lens), scale=0.1,
                               softcap=30.0 if sinks is not None else None,
                               sinks=None if sinks is None else sinks.cuda()).float().cpu().numpy()
    cells = gpu.view(torch.uint8).cpu().numpy()
    for b, (n, q) in enumerate(zip(lens, qlens)):
        if q == 0:
            continue
        k, v = oc.read_cells(gathered_cells(cells, table, b, n, page, layout), layout, NAMES[dtype])
        mask = np.zeros((1, 1, q, n), bool)
        for i in range(q):
            mask[..., i, : n - q + i + 1] = True
        qb = query[qsl[b]: qsl[b + 1]].float().numpy().transpose(1, 0, 2)[None]
        want = reference_attention(qb, k[None], v[None], mask, 0.1, 30.0 if sinks is not None else None,
                                   None if sinks is None else sinks.numpy())[0]
        np.testing.assert_allclose(out[qsl[b]: qsl[b + 1]], want, atol=2e-3, rtol=1e-2, err_msg=f"request {b}")


@pytest.mark.parametrize("bits", [2, 4])
def test_attention_reads_the_codes_of_quantized_cells(bits) -> None:
    """bf16 cells of 128 channels in key groups of 32 are attended through their codes wherever a flag is 1, as the
    reference's kernel reads them (kernels.py:274-296): with the dense entries of every quantized cell poisoned (NaN)
    the output still equals the oracle's read_cells definition. A group flagged as overflowed (2) and a cell whose
    flags were cleared (0), both holding their full-precision dense entries, are read from those entries."""
    from economize_amd.vllm_kivi import paged_kivi_attention
    from oracle.attention import reference_attention

    dtype, group, head, q_heads, page = torch.bfloat16, 32, 128, 8, 32
    residual = 2 * group
    lens = [9 * group + 7, 4 * group + 1, 6 * group, 3 * group + 3, 20 * group + 5]
    qlens = [1, 4, 2, 3, 1]
    layout, cache, table, states = setup(dtype, bits, group, head, page, lens, seed=40 + bits)
    gpu = cache.cuda()
    run(gpu, layout, residual, table, qlens, lens, [0] * len(lens))
    u8 = gpu.view(torch.uint8).cpu().numpy().copy()
    nan = np.array([0x7FC0], np.uint16).view(np.uint8)  # bf16 quiet NaN, little-endian bytes
    kflag = u8[..., layout.off_flag]
    vflag = u8[..., layout.off_flag + 1]
    assert (kflag == oc.FLAG_PACKED).sum() > 0 and (vflag == oc.FLAG_PACKED).sum() > 0
    k_entries = u8[..., : layout.off_v].reshape(*u8.shape[:3], head, 2)
    v_entries = u8[..., layout.off_v: layout.off_vs].reshape(*u8.shape[:3], head, 2)
    k_entries[kflag == oc.FLAG_PACKED] = nan
    v_entries[vflag == oc.FLAG_PACKED] = nan
    u8[..., : layout.off_v] = k_entries.reshape(*u8.shape[:3], -1)
    u8[..., layout.off_v: layout.off_vs] = v_entries.reshape(*u8.shape[:3], -1)

    def restore(b, h, t, key_flag, value_flag):
        cell = u8[int(table[b, t // page]), h, t % page]
        k, v = states[b]
        cell[: layout.off_v] = k[h, t].contiguous().view(torch.uint8).numpy()
        cell[layout.off_v: layout.off_vs] = v[h, t].contiguous().view(torch.uint8).numpy()
        cell[layout.off_flag] = key_flag
        cell[layout.off_flag + 1] = value_flag

    for t in range(group, 2 * group):  # request 0, KV head 0: key group 1 as overflowed
        restore(0, 0, t, oc.FLAG_OVERFLOW, u8[int(table[0, t // page]), 0, t % page, layout.off_flag + 1])
        if u8[int(table[0, t // page]), 0, t % page, layout.off_flag + 1] == oc.FLAG_PACKED:
            cell = u8[int(table[0, t // page]), 0, t % page]
            cell[layout.off_v: layout.off_vs] = np.tile(nan, head)
    restore(4, 1, 70, 0, 0)  # request 4, KV head 1: a cleared cell inside a quantized group
    gpu = torch.from_numpy(u8).view(dtype).cuda()

    gen = torch.Generator().manual_seed(bits)
    query = torch.randn(sum(qlens), q_heads, head, generator=gen).to(dtype)
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32)
    out = paged_kivi_attention(query.cuda(), gpu, layout, table.cuda(), qsl.cuda(),
                               torch.tensor(lens, dtype=torch.int32).cuda(), max(qlens), max(lens),
                               scale=head ** -0.5).float().cpu().numpy()
    assert np.isfinite(out).all()
    for b, (n, q) in enumerate(zip(lens, qlens)):
        k, v = oc.read_cells(gathered_cells(u8, table, b, n, page, layout), layout, NAMES[dtype])
        mask = np.zeros((1, 1, q, n), bool)
        for i in range(q):
            mask[..., i, : n - q + i + 1] = True
        qb = query[qsl[b]: qsl[b + 1]].float().numpy().transpose(1, 0, 2)[None]
        want = reference_attention(qb, k[None], v[None], mask, head ** -0.5)[0]
        np.testing.assert_allclose(out[qsl[b]: qsl[b + 1]], want, atol=2e-3, rtol=1e-2, err_msg=f"request {b}")


def _poisoned_cells(requests, kv_heads, lens, bits, page, seed, residual=64, qlens=None):
    """A cache of random bf16 cells of 128 channels (groups of 32) built on the GPU, quantize_committed at the pass's
    schedule, then the dense entries of every quantized key and value set to NaN: only the codes path can read it."""
    from economize_amd.vllm_kivi import cell_layout

    head = 128
    layout = cell_layout(head, torch.bfloat16, bits, 32)
    per_row = max(-(-n // page) for n in lens)
    pages = requests * per_row + 7
    gen = torch.Generator(device="cuda").manual_seed(seed)
    table = torch.randperm(pages, generator=gen, device="cuda")[: requests * per_row].view(requests, per_row)
    table = table.to(torch.int32).contiguous()
    cache = (torch.randn(pages, kv_heads, page, layout.size // 2, generator=gen, device="cuda") * 2).to(torch.bfloat16)
    u8 = cache.view(torch.uint8)
    u8[..., layout.off_flag: layout.off_flag + 2] = 0
    qlens = qlens or [1] * requests
    run(cache, layout, residual, table.cpu(), qlens, lens, [0] * requests)
    nan = torch.tensor([0x7FC0], dtype=torch.int16).view(torch.bfloat16).cuda()
    typed = cache.view(pages, kv_heads, page, layout.size // 2)
    kflag = u8[..., layout.off_flag] == oc.FLAG_PACKED
    vflag = u8[..., layout.off_flag + 1] == oc.FLAG_PACKED
    assert int(kflag.sum()) > 0 and int(vflag.sum()) > 0
    k_entries = typed[..., :head]
    v_entries = typed[..., head: 2 * head]
    k_entries[kflag] = nan
    v_entries[vflag] = nan
    return layout, cache, table, qlens


def _check_requests(out, query, qsl, cache, layout, table, lens, qlens, page, scale, requests_to_check):
    from oracle.attention import reference_attention

    cells = cache.view(torch.uint8).cpu().numpy()
    tab = table.cpu()
    for b in requests_to_check:
        n, q = lens[b], qlens[b]
        k, v = oc.read_cells(gathered_cells(cells, tab, b, n, page, layout), layout, "bf16")
        mask = np.zeros((1, 1, q, n), bool)
        for i in range(q):
            mask[..., i, : n - q + i + 1] = True
        qb = query[qsl[b]: qsl[b + 1]].float().cpu().numpy().transpose(1, 0, 2)[None]
        want = reference_attention(qb, k[None], v[None], mask, scale)[0]
        np.testing.assert_allclose(out[qsl[b]: qsl[b + 1]], want, atol=2e-3, rtol=1e-2, err_msg=f"request {b}")


@pytest.mark.parametrize("bits", [2, 4])
def test_codes_path_with_single_splits_and_long_waves(bits) -> None:
    """2048 programs (8 requests x 8 KV heads x 32 blocks of 16 query rows: 64 queries of 8 heads per KV head) leave
    one split per program, so every wave walks its row's ~66 tiles: the two-buffer handover of the codes state
    between consecutive tiles and the page window's reload past 32 tiles both run, over cells whose quantized dense
    entries are NaN."""
    from economize_amd.vllm_kivi import paged_kivi_attention

    requests, kv_heads, q_heads, page = 8, 8, 64, 32
    lens = [2100, 2117, 2048, 2090, 2133, 2101, 2060, 2111]
    qlens = [64, 64, 50, 64, 33, 64, 64, 64]
    layout, cache, table, qlens = _poisoned_cells(requests, kv_heads, lens, bits, page, seed=bits, qlens=qlens)
    gen = torch.Generator().manual_seed(bits)
    query = torch.randn(sum(qlens), q_heads, 128, generator=gen).to(torch.bfloat16)
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32)
    out = paged_kivi_attention(query.cuda(), cache, layout, table, qsl.cuda(),
                               torch.tensor(lens, dtype=torch.int32).cuda(), max(qlens), max(lens),
                               scale=128 ** -0.5).float().cpu().numpy()
    assert np.isfinite(out).all()
    _check_requests(out, query, qsl, cache, layout, table, lens, qlens, page, 128 ** -0.5, [0, 2, 4, 7])


@pytest.mark.parametrize("bits", [2, 4])
def test_codes_path_at_the_benchmark_shape(bits) -> None:
    """The measured cells workload: 16 requests of 8192 tokens, 32 query heads over 8 KV heads, one query each,
    residual 128, every quantized dense entry NaN; sampled requests against read_cells and the fp32 definition."""
    from economize_amd.vllm_kivi import paged_kivi_attention

    requests, kv_heads, q_heads, page, length = 16, 8, 32, 32, 8192
    lens = [length] * requests
    layout, cache, table, qlens = _poisoned_cells(requests, kv_heads, lens, bits, page, seed=10 + bits, residual=128)
    gen = torch.Generator().manual_seed(bits)
    query = torch.randn(requests, q_heads, 128, generator=gen).to(torch.bfloat16)
    qsl = torch.arange(requests + 1, dtype=torch.int32)
    out = paged_kivi_attention(query.cuda(), cache, layout, table, qsl.cuda(),
                               torch.tensor(lens, dtype=torch.int32).cuda(), 1, length,
                               scale=128 ** -0.5).float().cpu().numpy()
    assert np.isfinite(out).all()
    _check_requests(out, query, qsl, cache, layout, table, lens, qlens, page, 128 ** -0.5, [0, 9])
