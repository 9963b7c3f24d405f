"""Parity of the dense decode-attention kernel (economize_amd.decode.decode_attention, the reference's
decode_attention, attention/decode.py:252-324) with the fp32 definition (attention/decode.py:66-103, the oracle's
reference_attention) on the GPU: bf16 / fp16 / fp32 queries and K/V, fp8 K/V views (with and without per-head
scales), boolean masks broadcast over heads or per head, causal draft masks, rows that see nothing, sinks, soft caps,
more than 16 query rows per KV head, head dims 64 / 96 / 128 / 256, heads wider than 256 (up to 512) and Dv != D, the HF query layout
([B, Q, Hq, D].transpose(1, 2)), key counts that are not multiples of the tile. Tolerance atol 2e-3 / rtol 1e-2."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle.attention import reference_attention

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
FP8 = {torch.float8_e4m3fn: "e4m3", torch.float8_e5m2: "e5m2"}


def _case(batch, q_heads, kv_heads, queries, keys, d, dv, qdtype, kvdtype, seed, mask_kind=None, scaled=False):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, queries, q_heads, d, generator=gen).to(qdtype).transpose(1, 2)  # HF layout
    k32 = torch.randn(batch, kv_heads, keys, d, generator=gen)
    v32 = torch.randn(batch, kv_heads, keys, dv, generator=gen)
    ks = vs = None
    if kvdtype in FP8:
        fmt = FP8[kvdtype]
        if scaled:
            ks = ofp8.head_scales(k32.numpy(), fmt)
            vs = ofp8.head_scales(v32.numpy(), fmt)
        kc = ofp8.fp8_encode(k32.numpy(), fmt, None if ks is None else ks.reshape(1, -1, 1, 1))
        vc = ofp8.fp8_encode(v32.numpy(), fmt, None if vs is None else vs.reshape(1, -1, 1, 1))
        k = torch.from_numpy(kc).view(kvdtype)
        v = torch.from_numpy(vc).view(kvdtype)
        kf = ofp8.fp8_decode(kc, fmt, None if ks is None else ks.reshape(1, -1, 1, 1), "f32")
        vf = ofp8.fp8_decode(vc, fmt, None if vs is None else vs.reshape(1, -1, 1, 1), "f32")
    else:
        k, v = k32.to(kvdtype), v32.to(kvdtype)
        kf, vf = k.float().numpy(), v.float().numpy()
    rng = np.random.default_rng(seed)
    mask = None
    if mask_kind == "holes":
        mask = rng.random((batch, 1, 1, keys)) < 0.7
    elif mask_kind == "per_head":
        mask = rng.random((batch, q_heads, queries, keys)) < 0.6
    elif mask_kind == "causal":  # the last `queries` keys are the draft: query qi sees keys < keys - Q + qi + 1
        mask = np.zeros((batch, 1, queries, keys), bool)
        for qi in range(queries):
            mask[:, :, qi, : keys - queries + qi + 1] = True
    elif mask_kind == "window":
        mask = np.zeros((batch, 1, queries, keys), bool)
        mask[..., max(0, keys - 300):] = True
    elif mask_kind == "empty_row":
        mask = rng.random((batch, 1, queries, keys)) < 0.5
        mask[0] = False
    return q, k, v, kf, vf, mask, ks, vs


CASES = [
    # batch, Hq, Hkv, Q, keys, D, Dv, query dtype, K/V dtype, mask, per-head scales
    (3, 32, 8, 1, 1000, 128, 128, torch.bfloat16, torch.bfloat16, None, False),
    (2, 32, 8, 1, 777, 128, 128, torch.bfloat16, torch.float8_e4m3fn, "holes", False),
    (2, 16, 4, 1, 500, 128, 128, torch.bfloat16, torch.float8_e5m2, "holes", True),
    (2, 8, 2, 4, 300, 64, 64, torch.float16, torch.float16, "causal", False),
    (2, 8, 4, 2, 129, 96, 64, torch.float32, torch.float32, "per_head", False),
    (1, 32, 2, 3, 1500, 128, 128, torch.bfloat16, torch.bfloat16, "causal", False),  # 48 rows per KV head
    (2, 8, 8, 1, 2000, 256, 256, torch.bfloat16, torch.bfloat16, "window", False),
    (2, 16, 4, 2, 77, 64, 64, torch.float16, torch.float8_e4m3fn, "empty_row", False),
    (1, 4, 1, 1, 1, 128, 128, torch.bfloat16, torch.bfloat16, None, False),
    (2, 4, 2, 1, 300, 16, 16, torch.float32, torch.float8_e4m3fn, None, False),  # the golden model's head dim
    (2, 8, 2, 2, 333, 48, 48, torch.bfloat16, torch.bfloat16, "causal", False),
    (2, 12, 4, 1, 3000, 128, 128, torch.float32, torch.float8_e4m3fn, "holes", True),
    # heads wider than 256: two value slices of 256 channels (or one, Dv <= 256)
    (2, 8, 2, 1, 1000, 512, 512, torch.bfloat16, torch.bfloat16, None, False),
    (2, 8, 4, 2, 700, 512, 512, torch.float16, torch.float16, "causal", False),
    (1, 8, 1, 1, 2500, 512, 512, torch.float32, torch.float8_e4m3fn, "holes", True),
    (2, 16, 4, 3, 333, 320, 320, torch.bfloat16, torch.float8_e5m2, "per_head", False),
    (2, 8, 2, 1, 129, 384, 256, torch.bfloat16, torch.bfloat16, "empty_row", False),
    (2, 4, 2, 1, 100, 264, 512, torch.float16, torch.float16, None, False),  # Dv above D
    (1, 40, 2, 1, 5000, 512, 512, torch.bfloat16, torch.bfloat16, "window", False),  # 20 rows per KV head, splits
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}h{c[1]}k{c[2]}q{c[3]}s{c[4]}d{c[5]}v{c[6]}-"
                                             f"{str(c[7])[6:]}-{str(c[8])[6:]}-{c[9]}" for c in CASES])
def test_decode_matches_the_definition(case) -> None:
    from economize_amd.decode import decode_attention

    batch, hq, hkv, queries, keys, d, dv, qdt, kvdt, mask_kind, scaled = case
    q, k, v, kf, vf, mask, ks, vs = _case(batch, hq, hkv, queries, keys, d, dv, qdt, kvdt, seed=keys + d,
                                          mask_kind=mask_kind, scaled=scaled)
    m = None if mask is None else torch.from_numpy(mask).cuda()
    got = decode_attention(q.cuda(), k.cuda(), v.cuda(), m, 1 / np.sqrt(d),
                           k_scale=None if ks is None else torch.from_numpy(ks).cuda(),
                           v_scale=None if vs is None else torch.from_numpy(vs).cuda())
    assert got.dtype == qdt and got.shape == (batch, queries, hq, dv)
    want = reference_attention(q.float().numpy(), kf, vf, mask, 1 / np.sqrt(d))
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    if mask_kind == "empty_row":
        assert (got[0].float() == 0).all()


def test_softcap_and_sinks() -> None:
    from economize_amd.decode import decode_attention

    q, k, v, kf, vf, mask, _, _ = _case(2, 16, 4, 2, 600, 128, 128, torch.bfloat16, torch.bfloat16, seed=3,
                                        mask_kind="empty_row")
    sinks = np.random.default_rng(4).standard_normal(16).astype(np.float32)
    got = decode_attention(q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(mask).cuda(), 0.2, softcap=5.0,
                           sinks=torch.from_numpy(sinks).cuda())
    want = reference_attention(q.float().numpy(), kf, vf, mask, 0.2, softcap=5.0, sinks=sinks)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


def test_wide_heads_with_softcap_and_sinks() -> None:
    from economize_amd.decode import decode_attention

    q, k, v, kf, vf, mask, _, _ = _case(2, 8, 2, 2, 900, 512, 512, torch.bfloat16, torch.bfloat16, seed=5,
                                        mask_kind="empty_row")
    sinks = np.random.default_rng(6).standard_normal(8).astype(np.float32)
    got = decode_attention(q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(mask).cuda(), 0.05, softcap=4.0,
                           sinks=torch.from_numpy(sinks).cuda())
    want = reference_attention(q.float().numpy(), kf, vf, mask, 0.05, softcap=4.0, sinks=sinks)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


def test_refusals() -> None:
    from economize_amd.decode import decode_attention
    from economize_amd.errors import ConfigError

    q = torch.zeros(1, 6, 1, 64, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(1, 4, 10, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ConfigError, match="multiple"):
        decode_attention(q, k, k, None, 1.0)
    with pytest.raises(ConfigError, match="does not match"):
        decode_attention(q[:, :4], k.half(), k.half(), None, 1.0)
    with pytest.raises(ConfigError, match="boolean"):
        decode_attention(q[:, :4], k, k, torch.ones(1, 1, 1, 10, device="cuda"), 1.0)
    with pytest.raises(ConfigError, match="keys"):
        decode_attention(q[:, :4], k, k, torch.ones(1, 1, 1, 11, dtype=torch.bool, device="cuda"), 1.0)
    wide = torch.zeros(1, 4, 1, 512, dtype=torch.float32, device="cuda")
    with pytest.raises(ConfigError, match="256 for fp32"):  # fp32 K/V: heads up to 256
        decode_attention(wide, wide, wide, None, 1.0)
    with pytest.raises(ConfigError, match="up to 512"):
        decode_attention(torch.zeros(1, 4, 1, 528, dtype=torch.bfloat16, device="cuda"),
                         torch.zeros(1, 4, 1, 528, dtype=torch.bfloat16, device="cuda"),
                         torch.zeros(1, 4, 1, 528, dtype=torch.bfloat16, device="cuda"), None, 1.0)


def sweep_case(i: int):
    """Randomized dense decode case ``i``: query and K/V dtypes (fp8 views with or without per-head scales), head dims
    (D and Dv apart), GQA, query count, key count and mask kind, drawn from a seeded generator on the CPU."""
    rng = np.random.default_rng(70_000 + i)
    qdt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    kvdt = [qdt, qdt, torch.float8_e4m3fn, torch.float8_e5m2][int(rng.integers(0, 4))]
    d = int(rng.choice([16, 48, 64, 96, 128, 256]))
    dv = d if rng.random() < 0.8 else int(rng.choice([32, 64, 128]))
    if kvdt in FP8:  # fp8 rows are multiples of 16 bytes
        d, dv = max(16, d // 16 * 16), max(16, dv // 16 * 16)
    hkv = int(rng.choice([1, 2, 4, 8]))
    groups = int(rng.choice([1, 2, 4, 8]))
    queries = int(rng.integers(1, 5))
    keys = int(rng.choice([1, 31, 33, 200, 1000, 2500]))
    mask_kind = [None, "holes", "per_head", "causal", "empty_row"][int(rng.integers(0, 5))]
    if mask_kind == "causal" and keys < queries:
        mask_kind = None
    scaled = kvdt in FP8 and rng.random() < 0.5
    return int(rng.integers(1, 4)), groups * hkv, hkv, queries, keys, d, dv, qdt, kvdt, mask_kind, scaled, 80_000 + i


SWEEP = [sweep_case(i) for i in range(150)]


@pytest.mark.parametrize("case", SWEEP, ids=[f"{i}-b{c[0]}h{c[1]}k{c[2]}q{c[3]}s{c[4]}d{c[5]}v{c[6]}-"
                                             f"{str(c[7])[6:]}-{str(c[8])[6:]}-{c[9]}" for i, c in enumerate(SWEEP)])
def test_randomized_sweep(case) -> None:
    from economize_amd.decode import decode_attention

    batch, hq, hkv, queries, keys, d, dv, qdt, kvdt, mask_kind, scaled, seed = case
    q, k, v, kf, vf, mask, ks, vs = _case(batch, hq, hkv, queries, keys, d, dv, qdt, kvdt, seed=seed,
                                          mask_kind=mask_kind, scaled=scaled)
    m = None if mask is None else torch.from_numpy(mask).cuda()
    got = decode_attention(q.cuda(), k.cuda(), v.cuda(), m, 1 / np.sqrt(d),
                           k_scale=None if ks is None else torch.from_numpy(ks).cuda(),
                           v_scale=None if vs is None else torch.from_numpy(vs).cuda())
    want = reference_attention(q.float().numpy(), kf, vf, mask, 1 / np.sqrt(d))
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
