"""The registered ``"economize"`` forward on the GPU: every cache format it dispatches to gives the oracle's output
(within atol 2e-3 / rtol 1e-2), the softcap and sinks arrive through ``kwargs`` as the reference's forward reads them
(attention/interface.py:179-184), and Quest pages route a single query to the page-sparse kernel and a longer one to
dense attention (attention/quest.py:191-204)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import test_gpu_kivi as kivi_cases
from paged_cases import make_case, oracle_output

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _forward():
    from economize_amd.attention import ATTENTION_KERNELS

    return ATTENTION_KERNELS["economize"].forward


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.bfloat16])
def test_paged_formats(dtype) -> None:
    from economize_amd.attention import PagedKV, kernel_usage

    lens = [700, 1300]
    c = make_case(2, 1, 16, 4, 128, lens, dtype, seed=3)
    kv = PagedKV(c.device_cache(), torch.from_numpy(c.table).cuda(), torch.tensor(lens, dtype=torch.int32).cuda(),
                 max(lens))
    sinks = np.random.default_rng(2).standard_normal(16).astype(np.float32)
    kernel_usage(reset=True)
    out, weights = _forward()(None, c.q.cuda().transpose(1, 2), kv, None, None, scaling=0.1, softcap=5.0,
                              s_aux=torch.from_numpy(sinks).cuda())
    assert weights is None and out.shape == (2, 1, 16, 128)
    assert [(r["path"], r["calls"]) for r in kernel_usage(reset=True)] == [(f"kernel_{kv.format}", 1)]
    np.testing.assert_allclose(out.float().cpu().numpy(), oracle_output(c, 0.1, 5.0, sinks), atol=ATOL, rtol=RTOL)


def test_kivi_format() -> None:
    from economize_amd.attention import PagedKV

    c = kivi_cases.make_case(2, 1, 16, 4, 128, [900, 260], 2, seed=8)
    cache, table = kivi_cases.device_cache(c)
    kv = PagedKV(cache, table, torch.tensor(c.lens, dtype=torch.int32).cuda(), max(c.lens))
    assert kv.format == "kivi"
    out, _ = _forward()(None, c.q.cuda().transpose(1, 2), kv, None, None)
    np.testing.assert_allclose(out.float().cpu().numpy(), kivi_cases.oracle_output(c), atol=ATOL, rtol=RTOL)


def test_quest_format_routes_by_query_length() -> None:
    from economize_amd.attention import PagedKV
    from economize_amd.paged import paged_decode_attention
    from economize_amd.quest import QuestPages, paged_page_bounds

    lens = [2000, 1500]
    c = make_case(2, 1, 16, 4, 128, lens, torch.bfloat16, seed=12)
    cache = c.device_cache()
    table = torch.from_numpy(c.table).cuda()
    seq = torch.tensor(lens, dtype=torch.int32).cuda()
    done = np.array([(n - 1) // 16 for n in lens], np.int32)
    kmin, kmax = paged_page_bounds(cache, table, 0, int(done.max()), 16)
    qp = QuestPages(kmin, kmax, torch.from_numpy(done).cuda(), int(done.min()), int(done.max()), 16, 31)
    kv = PagedKV(cache, table, seq, max(lens), qp)
    assert kv.format == "quest"
    query = c.q.cuda().transpose(1, 2)
    out, _ = _forward()(None, query, kv, None, None)
    assert torch.equal(out, qp.attend_paged(query, cache, table, seq, max(lens)))
    # two queries per row exceed max_queries: dense attention over every key
    c2 = make_case(2, 2, 16, 4, 128, lens, torch.bfloat16, seed=12)
    query2 = c2.q.cuda().transpose(1, 2)
    out2, _ = _forward()(None, query2, PagedKV(c2.device_cache(), table, seq, max(lens), qp), None, None)
    dense = paged_decode_attention(c2.q.cuda(), c2.device_cache(), table, seq, max(lens))
    assert torch.equal(out2, dense)
    np.testing.assert_allclose(out2.float().cpu().numpy(), oracle_output(c2), atol=ATOL, rtol=RTOL)
