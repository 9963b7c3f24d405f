"""Quest metadata kept on append with every count on the device (``QuestState``, ``eco_quest_refresh_bounds``):
the bounds of committed pages equal the oracle's page_bounds as rows grow by single tokens and by jumps
(techniques/quest/technique.py:229-259: pages below ``done`` are final once computed), ``done`` follows
``committed // page``, the selection with the static ``max_done`` equals the one with the batch's true maximum, and
a whole decode step (append, bounds refresh, selection, page-list attention) captured in a HIP graph gives the eager
result at every replay while the rows grow; the append that refreshes the bounds in its own launch
(``eco_paged_append_quest``) equals the append and the refresh as two launches."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quest as oquest

pytestmark = pytest.mark.gpu

B, HKV, HQ, D, CAP = 3, 2, 8, 128, 640  # CAP tokens per row


def make_cache(dtype, seed: int):
    from economize_amd.paged import PagedKVCache, paged_append

    gen = torch.Generator().manual_seed(seed)
    per_row = CAP // 16
    cache = PagedKVCache.empty(B * per_row + 5, HKV, D, dtype, "cuda")
    perm = torch.randperm(B * per_row + 5, generator=gen)[: B * per_row].view(B, per_row).to(torch.int32)
    table = perm.cuda()
    keys = torch.randn(B, HKV, CAP, D, generator=gen).to(torch.bfloat16)
    values = torch.randn(B, HKV, CAP, D, generator=gen).to(torch.bfloat16)
    pos = torch.arange(CAP)
    slots = (perm[:, pos // 16] * 16 + pos % 16).reshape(-1).to(torch.int32).cuda()
    paged_append(cache, keys.transpose(1, 2).reshape(B * CAP, HKV, D).cuda(),
                 values.transpose(1, 2).reshape(B * CAP, HKV, D).cuda(), slots)
    return cache, table, keys, values


def stored_keys(keys: torch.Tensor, dtype) -> np.ndarray:
    """The key values the cache holds (fp8 codes decoded exactly)."""
    return keys.to(dtype).float().numpy() if dtype != torch.bfloat16 else keys.float().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("page", [16, 32])
def test_refresh_keeps_the_committed_bounds_of_the_oracle(dtype, page) -> None:
    from economize_amd.quest import QuestState

    cache, table, keys, _ = make_cache(dtype, seed=page)
    ref = stored_keys(keys, dtype)
    state = QuestState(B, HKV, D, CAP // page, page, 3, "cuda")
    committed = np.zeros(B, np.int64)
    schedule = [(5, 0, 17), (1, 1, 1), (11, 40, 2), (16, 31, 1), (200, 1, 64), (1, 1, 1), (300, 500, 250)]
    for grow in schedule:
        committed = np.minimum(committed + np.array(grow), CAP)
        state.refresh(cache, table, torch.tensor(committed, dtype=torch.int32).cuda())
        done = committed // page
        assert state.done.cpu().numpy().tolist() == done.tolist()
        assert state.valid.view(B, HKV).cpu().numpy().tolist() == [[int(d)] * HKV for d in done]
        kmin, kmax = state.kmin.float().cpu().numpy(), state.kmax.float().cpu().numpy()
        for b in range(B):
            lo, hi = oquest.page_bounds(ref[b: b + 1], 0, int(done[b]), page)
            assert np.array_equal(kmin[b, :, : done[b]], lo[0]) and np.array_equal(kmax[b, :, : done[b]], hi[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("page", [16, 32])
def test_the_append_with_the_refresh_equals_the_two_launches(dtype, page) -> None:
    """eco_paged_append_quest (one launch) against eco_paged_append + eco_quest_refresh_bounds on a twin cache: the
    same cache bytes, bounds, valid pages and done at every step, with the counters left zero, while rows grow by
    single tokens, by jumps (a prompt's pages at once) and not at all (a refresh with nothing appended)."""
    from economize_amd.paged import paged_append
    from economize_amd.quest import QuestState

    (c0, t0, keys, values), (c1, t1, _, _) = make_cache(dtype, seed=3 + page), make_cache(dtype, seed=3 + page)
    assert torch.equal(t0, t1)
    s0 = QuestState(B, HKV, D, CAP // page, page, 3, "cuda")
    s1 = QuestState(B, HKV, D, CAP // page, page, 3, "cuda")
    gen = torch.Generator().manual_seed(page)
    committed = np.zeros(B, np.int64)
    tab = t0.cpu()
    for step, grow in enumerate([(0, 0, 0), (70, 3, 200), (1, 1, 1), (0, 0, 0), (40, 300, 5), (16, 16, 16)]):
        committed = np.minimum(committed + np.array(grow), CAP - 1)
        tokens = step % 3  # new tokens per row at positions committed .. (the tokens of this pass)
        pos = [[min(int(committed[b]) + i, CAP - 1) for i in range(tokens)] for b in range(B)]
        slots = torch.tensor([int(tab[b, p // 16]) * 16 + p % 16 for b in range(B) for p in pos[b]],
                             dtype=torch.int32).cuda()
        k_new = torch.randn(B * tokens, HKV, D, generator=gen).to(torch.bfloat16).cuda()
        v_new = torch.randn(B * tokens, HKV, D, generator=gen).to(torch.bfloat16).cuda()
        lens = torch.tensor(committed, dtype=torch.int32).cuda()
        paged_append(c0, k_new, v_new, slots)
        s0.refresh(c0, t0, lens)
        s1.append(c1, k_new, v_new, slots, t1, lens)
        torch.cuda.synchronize()
        assert torch.equal(c0.keys, c1.keys) and torch.equal(c0.values, c1.values), step
        for name in ("kmin", "kmax", "valid", "done"):
            assert torch.equal(getattr(s0, name), getattr(s1, name)), (step, name)
        assert int(s1.counters.abs().sum()) == 0
    assert s1.done.cpu().tolist() == (committed // page).tolist()


def test_static_max_done_selects_as_the_true_maximum() -> None:
    from economize_amd.quest import QuestState, select_pages

    cache, table, keys, _ = make_cache(torch.bfloat16, seed=4)
    state = QuestState(B, HKV, D, CAP // 16, 16, 5, "cuda")
    committed = torch.tensor([600, 130, 77], dtype=torch.int32).cuda()  # done 37, 8, 4 (the last: fewer than 5)
    state.refresh(cache, table, committed)
    query = torch.randn(B, HQ, 1, D, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).cuda()
    got = select_pages(query, state.kmin, state.kmax, state.done, state.max_pages, state.pages)
    want = select_pages(query, state.kmin, state.kmax, state.done, 37, state.pages)
    assert torch.equal(got, want)
    oracle = oquest.select_pages(query.float().cpu().numpy(), state.kmin.float().cpu().numpy(),
                                 state.kmax.float().cpu().numpy(), np.array([37, 8, 4]), 37, 5)
    assert np.array_equal(got.cpu().numpy(), oracle)
    assert got[2].cpu().tolist() == [[0, 1, 2, 3, -1]] * HKV


@pytest.mark.parametrize("fused", [False, True])
def test_a_captured_quest_decode_step_replays_like_the_eager_one(fused: bool) -> None:
    """Each replay appends one token per row, refreshes the bounds (in the append's launch when fused), selects and
    attends, all from device buffers filled between replays (the graph holds no host count); an identical eager
    pipeline on a twin cache gives the same bits at every step, across page boundaries of every row."""
    from economize_amd.paged import paged_append
    from economize_amd.quest import QuestState, paged_quest_decode_attention

    page, pages = 16, 3
    caches, states = [], []
    lens0 = torch.tensor([100, 63, 47], dtype=torch.int32)
    for _ in range(2):
        cache, table, keys, values = make_cache(torch.bfloat16, seed=21)
        state = QuestState(B, HKV, D, CAP // page, page, pages, "cuda")
        state.refresh(cache, table, lens0.cuda())
        caches.append((cache, table))
        states.append(state)
    gen = torch.Generator().manual_seed(5)
    # static inputs of the captured step
    q = torch.zeros(B, 1, HQ, D, dtype=torch.bfloat16, device="cuda")
    k_new = torch.zeros(B, HKV, D, dtype=torch.bfloat16, device="cuda")
    v_new = torch.zeros(B, HKV, D, dtype=torch.bfloat16, device="cuda")
    slots = torch.zeros(B, dtype=torch.int32, device="cuda")
    committed = torch.zeros(B, dtype=torch.int32, device="cuda")
    seq_lens = torch.zeros(B, dtype=torch.int32, device="cuda")
    out = torch.zeros(B, 1, HQ, D, dtype=torch.bfloat16, device="cuda")

    def step(cache, table, state, out_buf):
        if fused:
            state.append(cache, k_new, v_new, slots, table, committed)
        else:
            paged_append(cache, k_new, v_new, slots)
            state.refresh(cache, table, committed)
        paged_quest_decode_attention(q.transpose(1, 2), cache, table, seq_lens, CAP, state.pages_handle(),
                                     out=out_buf)

    def fill(length: torch.Tensor, table: torch.Tensor) -> None:
        q.copy_(torch.randn(B, 1, HQ, D, generator=gen).to(torch.bfloat16))
        k_new.copy_(torch.randn(B, HKV, D, generator=gen).to(torch.bfloat16))
        v_new.copy_(torch.randn(B, HKV, D, generator=gen).to(torch.bfloat16))
        tab = table.cpu()
        slots.copy_(torch.tensor([int(tab[b, int(length[b]) // 16]) * 16 + int(length[b]) % 16 for b in range(B)],
                                 dtype=torch.int32))
        committed.copy_(length)
        seq_lens.copy_(length + 1)

    (c0, t0), (c1, t1) = caches
    lens = lens0.clone()
    fill(lens, t0)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream: workspaces exist before capture
        step(c1, t1, states[1], out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # the warm-up wrote step 0 into the twin: do the same eagerly for the captured cache's history
    step(c0, t0, states[0], torch.empty_like(out))
    torch.cuda.synchronize()
    lens += 1
    graph = torch.cuda.CUDAGraph()
    eager_out = torch.zeros_like(out)
    fill(lens, t0)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step(c0, t0, states[0], out)
    # capture records without running: the step for `lens` runs at the first replay below
    for i in range(40):
        if i:
            lens += 1
            fill(lens, t0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        step(c1, t1, states[1], eager_out)
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out), f"replay {i}, lengths {lens.tolist()}"
        assert torch.equal(states[0].done, states[1].done) and torch.equal(states[0].kmin, states[1].kmin)
    assert (lens // page).tolist() != (lens0 // page).tolist()  # rows crossed page boundaries
