"""eco_paged_decode_static (the decode entry point that allocates nothing: its scratch is a static device array of
the library) against eco_paged_decode with a workspace, through the C ABI: two calls in a row, the second smaller,
each bit-identical to the workspace entry point's output (the same kernels on the same inputs), and a call whose
workspace would exceed the array refused before any launch."""

from __future__ import annotations

import math

import pytest
import torch

from paged_cases import make_case

pytestmark = pytest.mark.gpu


def _args(case, cache, table, lens, out):
    from economize_amd import _lib

    q = case.q.cuda()
    batch, queries, q_heads, head_dim = q.shape
    return q, [
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        cache.keys.data_ptr(), cache.values.data_ptr(), _lib.fmt(cache.dtype), cache.num_pages,
        _lib.ptr(cache.k_scale), _lib.ptr(cache.v_scale),
        table.data_ptr(), table.stride(0), table.shape[1], lens.data_ptr(),
        None, 0, 0, 0, 16, None, None,
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        batch, queries, q_heads, cache.kv_heads, head_dim, 16, int(max(case.lens)), 1.0 / math.sqrt(head_dim), 0.0,
        None, 0, 0, 0, 0,
    ]


def _both(case):
    from economize_amd import _lib
    from economize_amd.paged import new_workspace, workspace_size

    cache = case.device_cache()
    table = torch.from_numpy(case.table).cuda()
    lens = torch.tensor(case.lens, dtype=torch.int32, device="cuda")
    out_ws = torch.full(tuple(case.q.shape), float("nan"), dtype=torch.bfloat16, device="cuda")
    out_st = torch.full_like(out_ws, float("nan"))
    q, args = _args(case, cache, table, lens, out_ws)
    batch, queries, q_heads, head_dim = q.shape
    need = workspace_size(batch, queries, q_heads, cache.kv_heads, head_dim, max(case.lens), 0, cache.dtype)
    ws = new_workspace(need, "cuda")
    stream = _lib.stream_of(q.device)
    _lib.call("eco_paged_decode", args[0], _lib.ECO_BF16, *args[1:], ws.data_ptr(), ws.numel(), stream)
    _, args = _args(case, cache, table, lens, out_st)
    _lib.call("eco_paged_decode_static", *args, stream)
    torch.cuda.synchronize()
    return out_ws.cpu(), out_st.cpu()


def test_static_scratch_matches_the_workspace_entry_point() -> None:
    big = make_case(32, 1, 32, 8, 128, [4096 - 37 * i for i in range(32)], torch.float8_e4m3fn, seed=3)
    small = make_case(3, 2, 16, 4, 128, [700, 65, 1300], torch.float8_e4m3fn, seed=4)
    for case in (big, small):
        got_ws, got_st = _both(case)
        assert not torch.isnan(got_st.float()).any()
        assert torch.equal(got_ws.view(torch.int16), got_st.view(torch.int16))


def test_a_call_beyond_the_scratch_is_refused() -> None:
    from economize_amd import _lib
    from economize_amd.errors import ConfigError

    case = make_case(2, 4, 64, 4, 256, [100, 90], torch.bfloat16, seed=5)  # 64 rows per KV head at head dim 256
    cache = case.device_cache()
    table = torch.from_numpy(case.table).cuda()
    lens = torch.tensor(case.lens, dtype=torch.int32, device="cuda")
    out = torch.zeros(tuple(case.q.shape), dtype=torch.bfloat16, device="cuda")
    q, args = _args(case, cache, table, lens, out)
    args[-8] = 1 << 20  # max_seq_len: a launch sized for a million tokens per row needs more scratch
    need = _lib.lib().eco_paged_decode_workspace_size(2, 4, 64, 4, 256, 1 << 20, 0, 16, _lib.ECO_BF16)
    assert need > 32 << 20
    with pytest.raises(ConfigError, match="more than the library's"):
        _lib.call("eco_paged_decode_static", *args, _lib.stream_of(q.device))
    torch.cuda.synchronize()
    assert not out.float().any()
