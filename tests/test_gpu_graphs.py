"""Decode calls captured in a HIP graph (``torch.cuda.graph``): every replay equals the eager call over the same inputs
bit for bit, with the inputs changed in place between replays and eager work in between. Nothing of a call is fixed
at capture but its launch shapes: the kernels read every length and count on the device and leave their workspace
counters zero, so one captured decode step serves every later step of the same shapes."""

from __future__ import annotations

import pytest
import torch

from paged_cases import make_case

pytestmark = pytest.mark.gpu


def _check_replays(graph_call, eager_call, out_graph: torch.Tensor, out_eager: torch.Tensor, change,
                   replays: int = 4) -> None:
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph_call()  # on the capture stream first: its cached workspace exists before the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        graph_call()
    for i in range(replays):
        change(i)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager_call()
        torch.cuda.synchronize()
        assert torch.isfinite(out_eager.float()).all(), f"replay {i}"
        assert torch.equal(out_graph, out_eager), f"replay {i}: {(out_graph.float() - out_eager.float()).abs().max()}"


@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16])
def test_paged_decode_replays(qdtype) -> None:
    """fp8 paged decode (bf16 queries, and fp16 queries with fp16 output), rows long enough to be cut between
    workgroups, their lengths shortened in place between replays."""
    from economize_amd.paged import new_workspace, paged_decode_attention, workspace_size

    lens = [3000, 17, 900, 1600, 2500, 1]
    smax = max(lens)
    c = make_case(len(lens), 1, 32, 8, 128, lens, torch.float8_e4m3fn, seed=5)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    q = c.q.to(qdtype).cuda()
    nbytes = workspace_size(len(lens), 1, 32, 8, 128, smax)
    ws_graph, ws_eager = new_workspace(nbytes, "cuda"), new_workspace(nbytes, "cuda")
    out_graph, out_eager = torch.empty_like(q), torch.empty_like(q)
    gen = torch.Generator().manual_seed(9)

    def change(i: int) -> None:
        q.copy_(torch.randn(q.shape, generator=gen).to(qdtype))
        seq.copy_(torch.tensor([max(1, n - 311 * i) for n in lens], dtype=torch.int32))

    print(f"graph: paged fp8 decode, {qdtype} queries", flush=True)
    _check_replays(lambda: paged_decode_attention(q, cache, table, seq, smax, out=out_graph, workspace=ws_graph),
                   lambda: paged_decode_attention(q, cache, table, seq, smax, out=out_eager, workspace=ws_eager),
                   out_graph, out_eager, change)


def test_kivi_decode_replays() -> None:
    """The paged KIVI decode (int2 codes, bf16 rings) over rows cut between workgroups."""
    from economize_amd.kivi import kivi_decode_attention
    from test_gpu_kivi import device_cache, make_case as kivi_case

    lens = [3000, 900, 40]
    c = kivi_case(len(lens), 1, 32, 8, 128, lens, 2, seed=11)
    cache, table = device_cache(c)
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    q = c.q.cuda()
    out_graph, out_eager = torch.empty_like(q), torch.empty_like(q)
    gen = torch.Generator().manual_seed(13)

    def change(i: int) -> None:
        q.copy_(torch.randn(q.shape, generator=gen).to(torch.bfloat16))

    print("graph: paged KIVI decode", flush=True)
    _check_replays(lambda: kivi_decode_attention(q, cache, table, seq, max(lens), out=out_graph),
                   lambda: kivi_decode_attention(q, cache, table, seq, max(lens), out=out_eager),
                   out_graph, out_eager, change)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kivi_packed_decode_replays(dtype) -> None:
    """The dense kernel's KIVI packed mode (the reference's layout, 4-bit codes, groups of 32)."""
    from economize_amd.kivi_packed import kivi_decode_attention
    from test_gpu_kivi_packed import BATCH, KEYS, KQ, KV_HEADS, Q_HEADS, VQ, _records

    gen = torch.Generator().manual_seed(17)
    key = torch.randn(BATCH, KV_HEADS, KEYS, 128, generator=gen).to(dtype)
    value = torch.randn(BATCH, KV_HEADS, KEYS, 128, generator=gen).to(dtype)
    packed, _, _, key_nan, value_nan = _records(key, value, 4, 32, KQ, VQ, "cuda")
    key_nan, value_nan = key_nan.cuda(), value_nan.cuda()
    q = torch.randn(BATCH, 1, Q_HEADS, 128, generator=gen).to(dtype).cuda().transpose(1, 2)  # [B, Hq, Q, D]
    out_graph = torch.empty(BATCH, 1, Q_HEADS, 128, dtype=dtype, device="cuda")
    out_eager = torch.empty_like(out_graph)
    scale = 128 ** -0.5

    def change(i: int) -> None:
        q.copy_(torch.randn(q.shape, generator=gen).to(dtype))

    print(f"graph: KIVI packed decode, {dtype}", flush=True)
    _check_replays(lambda: kivi_decode_attention(q, key_nan, value_nan, None, scale, packed, out=out_graph),
                   lambda: kivi_decode_attention(q, key_nan, value_nan, None, scale, packed, out=out_eager),
                   out_graph, out_eager, change)
