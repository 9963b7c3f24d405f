"""Decode attention over compacted prompt entries (``eco_gathered_decode``, the reference's
gathered_decode_attention, attention/gathered.py:96-179) against the oracle's virtual-axis attention, within atol
2e-3 / rtol 1e-2: compact entries read below each (row, KV head)'s count (the dense buffer's prompt slots and the
capacity past the count hold NaN, so reading either would show), dense slots from ``start[b]`` on, mask columns
through ``index``; GQA, bf16 / fp16 / fp32, ``Dv != D``, causal and per-head masks, soft cap, sinks, a row without
prompt entries, rows whose tail is empty; and the registered forward routes a key carrying a ``GatheredKV`` to the
kernel."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.gathered import gathered_reference

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def make(batch, q_heads, kv_heads, queries, slots, d, dv, dtype, seed, starts, mask_kind=None, capacity=None):
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    q = torch.randn(batch, q_heads, queries, d, generator=gen).to(dtype)
    k = torch.randn(batch, kv_heads, slots, d, generator=gen).to(dtype)
    v = torch.randn(batch, kv_heads, slots, dv, generator=gen).to(dtype)
    start = np.array(starts, np.int64)
    cap = capacity or max(int(start.max()), 1)
    ck = torch.full((batch, kv_heads, cap, d), float("nan")).to(dtype)
    cv = torch.full((batch, kv_heads, cap, dv), float("nan")).to(dtype)
    index = torch.zeros(batch, kv_heads, cap, dtype=torch.int32)
    count = torch.zeros(batch, kv_heads, dtype=torch.int32)
    for b in range(batch):
        for h in range(kv_heads):
            kept = np.nonzero(rng.random(int(start[b])) < rng.uniform(0.2, 0.8))[0]
            rows = torch.from_numpy(kept.astype(np.int64))
            count[b, h] = len(kept)
            ck[b, h, : len(kept)] = k[b, h, rows]
            cv[b, h, : len(kept)] = v[b, h, rows]
            index[b, h, : len(kept)] = rows.to(torch.int32)
    dropped = int(min(start[b] - count[b, h] for b in range(batch) for h in range(kv_heads)))
    mask = None
    if mask_kind == "causal":  # the last `queries` slots are the draft
        mask = np.zeros((batch, 1, queries, slots), bool)
        for qi in range(queries):
            mask[:, :, qi, : slots - queries + qi + 1] = True
    elif mask_kind == "per_head":
        mask = rng.random((batch, q_heads, queries, slots)) < 0.7
    k_poisoned, v_poisoned = k.clone(), v.clone()
    for b in range(batch):
        k_poisoned[b, :, : int(start[b])] = float("nan")
        v_poisoned[b, :, : int(start[b])] = float("nan")
    return dict(q=q, k=k, v=v, kp=k_poisoned, vp=v_poisoned, ck=ck, cv=cv, index=index, count=count,
                start=torch.from_numpy(start.astype(np.int32)), dropped=dropped, mask=mask)


def oracle(c, scale, softcap=None, sinks=None):
    f = lambda t: t.float().numpy()  # noqa: E731
    return gathered_reference(f(c["q"]), f(c["k"]), f(c["v"]), c["mask"], scale, f(c["ck"]), f(c["cv"]),
                               c["index"].numpy(), c["count"].numpy(), c["start"].numpy(), softcap, sinks)


def run(c, scale, softcap=None, sinks=None):
    from economize_amd.gathered import GatheredKV, gathered_decode_attention

    g = GatheredKV(c["ck"].cuda(), c["cv"].cuda(), c["index"].cuda(), c["count"].cuda(), c["start"].cuda(),
                   c["dropped"])
    mask = None if c["mask"] is None else torch.from_numpy(c["mask"]).cuda()
    s = None if sinks is None else torch.from_numpy(sinks).cuda()
    return gathered_decode_attention(c["q"].cuda(), c["kp"].cuda(), c["vp"].cuda(), mask, scale, g, softcap=softcap,
                                     sinks=s)


CASES = [  # batch, Hq, Hkv, Q, slots, D, Dv, dtype, starts, mask
    (2, 32, 8, 1, 700, 128, 128, torch.bfloat16, [500, 650], None),
    (3, 8, 2, 4, 333, 64, 64, torch.float16, [200, 0, 329], "causal"),
    (2, 16, 4, 2, 257, 96, 64, torch.float32, [100, 257], "per_head"),
    (1, 8, 8, 1, 1500, 256, 256, torch.bfloat16, [1400], None),
    (2, 4, 1, 3, 90, 128, 128, torch.bfloat16, [90, 45], "causal"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}h{c[1]}k{c[2]}q{c[3]}s{c[4]}d{c[5]}v{c[6]}-{c[9]}"
                                             for c in CASES])
def test_gathered_decode_matches_the_oracle(case) -> None:
    batch, hq, hkv, queries, slots, d, dv, dtype, starts, mask_kind = case
    c = make(batch, hq, hkv, queries, slots, d, dv, dtype, seed=slots, starts=starts, mask_kind=mask_kind)
    got = run(c, 1 / d ** 0.5).float().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, oracle(c, 1 / d ** 0.5), atol=ATOL, rtol=RTOL)


def test_softcap_and_sinks() -> None:
    c = make(2, 16, 4, 1, 400, 128, 128, torch.bfloat16, seed=7, starts=[300, 120], capacity=320)
    sinks = np.random.default_rng(1).standard_normal(16).astype(np.float32)
    got = run(c, 0.2, softcap=8.0, sinks=sinks).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle(c, 0.2, 8.0, sinks), atol=ATOL, rtol=RTOL)


def test_the_forward_routes_a_gathered_key_to_the_kernel() -> None:
    from economize_amd.attention import ATTENTION_KERNELS, kernel_usage
    from economize_amd.gathered import GatheredKV
    from economize_amd.packed import attach_packed

    c = make(2, 8, 2, 1, 300, 128, 128, torch.bfloat16, seed=3, starts=[250, 100])
    g = GatheredKV(c["ck"].cuda(), c["cv"].cuda(), c["index"].cuda(), c["count"].cuda(), c["start"].cuda(),
                   c["dropped"])
    key = attach_packed(c["kp"].cuda(), g)
    kernel_usage(reset=True)
    out, _ = ATTENTION_KERNELS["economize"].forward(None, c["q"].cuda(), key, c["vp"].cuda(), None, scaling=0.1)
    assert [(r["path"], r["calls"]) for r in kernel_usage(reset=True)] == [("kernel_gathered", 1)]
    np.testing.assert_allclose(out.float().cpu().numpy(), oracle(c, 0.1), atol=ATOL, rtol=RTOL)
