"""Parity of the KIVI packed decode (economize_amd.kivi_packed.kivi_decode_attention, the reference's
kivi_decode_attention over a KIVIPacked record, attention/kivi.py:199-309) on the GPU.

The codes, scales and zero points come from the oracle's quantizer and packer (oracle/kivi.py, pinned against the
reference's closed forms and golden tokens). The slots the codes cover are NaN in the dense buffers handed to the
kernel, so any read of them would show. The output must be bit-identical to the dense kernel
(economize_amd.decode.decode_attention) over buffers holding the dequantized values, the oracle's ``code * scale +
zero`` in fp32 rounded to the dtype (the criterion of the reference's own kernel test,
tests/unit/test_attention_kivi.py:1-7), and within atol 2e-3 / rtol 1e-2 of the oracle's fp32 attention. Cases: 2 / 4
/ 8 bits; bf16, fp16 and fp32; chain, tree and per-head masks; soft caps and sinks; key groups that split a 32-key tile
(16), hold one (128) or neither (24, 6); value groups of the whole head, of 16-byte chunks and smaller (per-element
scales); Dv != D; heads of 320 and 512 channels; full-precision entries from rings; rows with nothing quantized."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kivi as okivi
from oracle.attention import reference_attention

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
BATCH, Q_HEADS, KV_HEADS, KEYS = 3, 8, 2, 300
KQ, VQ = [256, 128, 0], [133, 12, 0]
FILLED = [260, 140, 30]


def _records(key: torch.Tensor, value: torch.Tensor, bits: int, group: int, kq, vq, device: str):
    """The packed record of ``key`` / ``value`` (cache dtype, CPU) and the dense buffers with the packed slots
    dequantized (``ok``) and NaN (``nan``)."""
    from economize_amd.kivi_packed import KIVIPacked

    b, h, s, d = key.shape
    dv = value.shape[3]
    vg = group if dv % group == 0 else dv
    full = s // group * group
    kf, vf = key.float().numpy(), value.float().numpy()
    pk, ks, kz, kdeq = okivi.quantize_keys(kf, 0, full, bits, group)
    pv, vs, vz, vdeq = okivi.quantize_values(vf, 0, s, bits, group)
    key_codes = np.zeros((b, h, s, d * bits // 8), np.uint8)
    key_codes[:, :, :full] = pk
    key_scale = np.zeros((b, h, -(-s // group), d), np.float16)
    key_zero = np.zeros_like(key_scale)
    key_scale[:, :, : full // group] = ks.astype(np.float16)
    key_zero[:, :, : full // group] = kz.astype(np.float16)
    k_deq = kf.copy()
    k_deq[:, :, :full] = kdeq
    k_deq = torch.from_numpy(k_deq).to(key.dtype)
    v_deq = torch.from_numpy(vdeq).to(value.dtype)
    slots = torch.arange(s)
    k_in = (slots[None, :] < torch.tensor(kq)[:, None])[:, None, :, None]
    v_in = (slots[None, :] < torch.tensor(vq)[:, None])[:, None, :, None]
    key_ok = torch.where(k_in, k_deq, key)
    value_ok = torch.where(v_in, v_deq, value)
    key_nan = key_ok.masked_fill(k_in, float("nan"))
    value_nan = value_ok.masked_fill(v_in, float("nan"))
    packed = KIVIPacked(
        bits=bits, key_group=group, value_group=vg,
        key_codes=torch.from_numpy(key_codes).to(device),
        key_scale=torch.from_numpy(key_scale).to(device), key_zero=torch.from_numpy(key_zero).to(device),
        value_codes=torch.from_numpy(pv).to(device),
        value_scale=torch.from_numpy(vs.astype(np.float16)).to(device),
        value_zero=torch.from_numpy(vz.astype(np.float16)).to(device),
        keys_quantized=torch.tensor(kq, dtype=torch.int32, device=device),
        values_quantized=torch.tensor(vq, dtype=torch.int32, device=device),
    )
    return packed, key_ok, value_ok, key_nan, value_nan


def _mask(kind: str | None, queries: int) -> torch.Tensor | None:
    """Boolean [B, 1 or Hq, Q, S]: "chain" (query i sees keys up to filled + i), "tree" (the drafted keys past the
    committed prefix are visible to queries of the same parity only, besides the query's own key), "per_head"
    (chain, and every other query head evicts keys 10..39)."""
    if kind is None:
        return None
    pos = torch.arange(KEYS)
    qpos = torch.tensor(FILLED)[:, None] + torch.arange(queries)[None, :]
    visible = pos[None, None, :] <= qpos[..., None]
    if kind == "tree":
        start = torch.tensor(FILLED)[:, None, None]
        drafted = (pos[None, None, :] >= start) & visible
        same = (pos[None, None, :] - start) % 2 == (torch.arange(queries)[None, :, None] % 2)
        visible &= ~drafted | same | (pos[None, None, :] == qpos[..., None])
    heads = Q_HEADS if kind == "per_head" else 1
    visible = visible[:, None].expand(BATCH, heads, queries, KEYS).clone()
    if heads > 1:
        visible[:, ::2, :, 10:40] = False
    return visible


CASES = [
    # bits, dtype, queries, mask, softcap, sinks, head dim, value head dim, group
    (2, torch.float32, 1, None, None, False, 64, 64, 32),
    (2, torch.bfloat16, 1, "chain", None, False, 128, 128, 32),
    (4, torch.bfloat16, 5, "chain", None, False, 128, 128, 32),
    (2, torch.bfloat16, 6, "tree", 30.0, False, 64, 64, 32),
    (8, torch.float16, 3, "per_head", None, True, 64, 64, 32),
    (4, torch.float32, 4, "tree", None, True, 128, 128, 32),
    (2, torch.bfloat16, 2, "chain", None, False, 64, 48, 32),  # value groups of the whole head (48 % 32 != 0)
    (2, torch.bfloat16, 3, "chain", None, False, 128, 128, 16),  # key groups that split a tile
    (4, torch.bfloat16, 3, "chain", None, False, 64, 64, 128),  # a key group over four tiles
    (2, torch.float16, 3, "chain", None, False, 48, 48, 24),  # groups that neither divide nor are divided by 32
    (8, torch.float32, 3, "chain", None, False, 64, 64, 16),
    (4, torch.bfloat16, 2, None, None, False, 48, 48, 12),  # value groups within a 16-byte chunk: per element
    (2, torch.float32, 1, "per_head", None, False, 48, 48, 6),
    (8, torch.bfloat16, 2, None, None, True, 64, 64, 4),
    (4, torch.float16, 2, "chain", None, True, 512, 512, 32),  # value slices of 256 channels
    (8, torch.bfloat16, 1, None, 20.0, False, 256, 256, 64),
    (2, torch.bfloat16, 1, None, None, False, 320, 320, 32),
    (4, torch.float32, 2, "chain", None, False, 256, 128, 32),
]


def _ids(c):
    return f"b{c[0]}-{str(c[1])[6:]}-q{c[2]}-{c[3]}-d{c[6]}v{c[7]}-g{c[8]}" + ("-cap" if c[4] else "") + \
        ("-sinks" if c[5] else "")


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_codes_match_dense_kernel_and_oracle(case) -> None:
    from economize_amd.decode import decode_attention
    from economize_amd.kivi_packed import kivi_decode_attention

    bits, dtype, queries, mask_kind, softcap, use_sinks, d, dv, group = case
    gen = torch.Generator().manual_seed(7 + bits + d)
    query = torch.randn(BATCH, queries, Q_HEADS, d, generator=gen).to(dtype).transpose(1, 2)  # HF layout
    key = torch.randn(BATCH, KV_HEADS, KEYS, d, generator=gen) * 2
    key[..., 3] += 20  # an outlier channel
    key = key.to(dtype)
    value = torch.randn(BATCH, KV_HEADS, KEYS, dv, generator=gen).to(dtype)
    packed, key_ok, value_ok, key_nan, value_nan = _records(key, value, bits, group, KQ, VQ, "cuda")
    mask = _mask(mask_kind, queries)
    sinks = torch.randn(Q_HEADS, generator=gen) if use_sinks else None
    scale = d ** -0.5
    dev = {"mask": None if mask is None else mask.cuda(), "softcap": softcap,
           "sinks": None if sinks is None else sinks.cuda()}
    print(f"kivi packed: {_ids(case)}", flush=True)
    got = kivi_decode_attention(query.cuda(), key_nan.cuda(), value_nan.cuda(), dev["mask"], scale, packed,
                                softcap=softcap, sinks=dev["sinks"])
    dense = decode_attention(query.cuda(), key_ok.cuda(), value_ok.cuda(), dev["mask"], scale, softcap=softcap,
                             sinks=dev["sinks"])
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got, dense), (got.float() - dense.float()).abs().max()
    want = reference_attention(query.float().numpy(), key_ok.float().numpy(), value_ok.float().numpy(),
                               None if mask is None else mask.numpy(), scale, softcap,
                               None if sinks is None else sinks.numpy())
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rings_hold_the_full_precision_entries(dtype) -> None:
    """``ring > 0``: the slots that are not packed come from the rings at ``s % ring`` (the reference's PackedKIVICache
    layout, techniques/kv_quant/packed.py:1-20); the dense K/V arguments are shape stand-ins."""
    from economize_amd.decode import decode_attention
    from economize_amd.kivi_packed import kivi_decode_attention

    keys, ring, d = 200, 64, 128
    kq, vq = [192, 160], [190, 150]
    gen = torch.Generator().manual_seed(3)
    query = torch.randn(2, 8, 1, d, generator=gen).to(dtype)
    key = (torch.randn(2, KV_HEADS, keys, d, generator=gen) * 3).to(dtype)
    value = torch.randn(2, KV_HEADS, keys, d, generator=gen).to(dtype)
    packed, key_ok, value_ok, _, _ = _records(key, value, 4, 32, kq, vq, "cuda")
    k_ring = torch.full((2, KV_HEADS, ring + 1, d), float("nan"), dtype=dtype)
    v_ring = torch.full((2, KV_HEADS, ring + 1, d), float("nan"), dtype=dtype)
    for s in range(keys - ring, keys):
        k_ring[:, :, s % ring] = key[:, :, s]
        v_ring[:, :, s % ring] = value[:, :, s]
    packed.key_ring, packed.value_ring, packed.ring = k_ring.cuda(), v_ring.cuda(), ring
    stand_k = torch.empty(2, KV_HEADS, keys, d, dtype=dtype, device="cuda")
    got = kivi_decode_attention(query.cuda(), stand_k, stand_k, None, d ** -0.5, packed)
    dense = decode_attention(query.cuda(), key_ok.cuda(), value_ok.cuda(), None, d ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(got, dense)


def test_rows_with_nothing_quantized_read_the_buffers() -> None:
    from economize_amd.decode import decode_attention
    from economize_amd.kivi_packed import kivi_decode_attention

    gen = torch.Generator().manual_seed(1)
    query = torch.randn(2, 4, 1, 64, generator=gen).to(torch.bfloat16).cuda()
    key = torch.randn(2, 2, 96, 64, generator=gen).to(torch.bfloat16)
    value = torch.randn(2, 2, 96, 64, generator=gen).to(torch.bfloat16)
    packed, *_ = _records(key, value, 2, 32, [0, 0], [0, 0], "cuda")
    got = kivi_decode_attention(query, key.cuda(), value.cuda(), None, 0.125, packed)
    assert torch.equal(got, decode_attention(query, key.cuda(), value.cuda(), None, 0.125))


def test_refusals() -> None:
    from economize_amd.errors import ConfigError
    from economize_amd.kivi_packed import kivi_decode_attention

    key = torch.randn(1, 2, 64, 64).to(torch.bfloat16)
    query = torch.randn(1, 4, 1, 64, dtype=torch.bfloat16, device="cuda")
    packed, *_ = _records(key, key, 2, 32, [32], [32], "cuda")
    k = key.cuda()
    with pytest.raises(ConfigError, match="query's dtype"):
        kivi_decode_attention(query.float(), k, k, None, 0.125, packed)
    bad = type(packed)(**{**packed.__dict__, "bits": 3})
    with pytest.raises(ConfigError, match="bits=3"):
        kivi_decode_attention(query, k, k, None, 0.125, bad)
    bad = type(packed)(**{**packed.__dict__, "key_scale": packed.key_scale[:, :, :1]})
    with pytest.raises(ConfigError, match="key_scale"):
        kivi_decode_attention(query, k, k, None, 0.125, bad)
    bad = type(packed)(**{**packed.__dict__, "keys_quantized": packed.keys_quantized.cpu()})
    with pytest.raises(ConfigError, match="keys_quantized"):
        kivi_decode_attention(query, k, k, None, 0.125, bad)
    bad = type(packed)(**{**packed.__dict__, "ring": 16})
    with pytest.raises(ConfigError, match="key_ring"):
        kivi_decode_attention(query, k, k, None, 0.125, bad)


# ---- the packed record written by the GPU (eco_kivi_pack_quantize) ------------------------------------------------

PACK_CASES = [
    # bits, dtype, head dim, group
    (2, torch.bfloat16, 128, 32),
    (4, torch.bfloat16, 64, 16),
    (8, torch.float16, 64, 32),
    (2, torch.float16, 48, 24),
    (4, torch.float32, 64, 128),
    (8, torch.float32, 48, 12),
    (2, torch.bfloat16, 64, 4),
]


@pytest.mark.parametrize("case", PACK_CASES, ids=[f"b{c[0]}-{str(c[1])[6:]}-d{c[2]}-g{c[3]}" for c in PACK_CASES])
@pytest.mark.parametrize("ring", [0, 1])
def test_pack_quantize_matches_the_oracle(case, ring) -> None:
    """Codes, fp16 scales and zero points bit-exact with the oracle's quantize + pack_codes (the reference's
    FusedKIVICache._quantize_block layout), per-row ranges, from a dense buffer written back with the dequantized
    values, or from a ring (slot s at s % ring) left as it was."""
    from economize_amd.kivi_packed import KIVIPackedStore

    bits, dtype, d, group = case
    batch, heads = 2, 2
    slots = 3 * max(group, 32)
    gen = torch.Generator().manual_seed(bits * 100 + d + group)
    data = torch.randn(batch, heads, slots, d, generator=gen) * 3
    data[..., 1] += 15
    data = data.to(dtype)
    vg = group if d % group == 0 else d
    kstart, kstop = [0, group], [2 * group, 3 * group]
    vstart, vstop = [5, 0], [slots - 3, slots - 40]
    store = KIVIPackedStore(batch, heads, slots, d, d, bits, group, "cuda")
    width = 2 * max(group, 32) + 8  # ring slots: more than the longest key range
    if ring:  # a ring of `width` slots that holds each range's slots (and later ones) at s % width
        src_k = torch.full((batch, heads, width, d), float("nan"), dtype=dtype)
        src_v = src_k.clone()
        for b in range(batch):
            for s in range(kstart[b], kstop[b]):
                src_k[b, :, s % width] = data[b, :, s]
        src_k, src_v = src_k.cuda(), src_v.cuda()
    else:
        src_k, src_v = data.clone().cuda(), data.clone().cuda()
    rows = lambda x: torch.tensor(x, dtype=torch.int32, device="cuda")  # noqa: E731
    store.quantize(src_k, "k", rows(kstart), rows(kstop), 2 * group, write_back=not ring, ring=width if ring else 0)
    if not ring:
        store.quantize(src_v, "v", rows(vstart), rows(vstop), slots, write_back=True)
    torch.cuda.synchronize()
    assert int(store.overflow.item()) == 0
    f = data.float().numpy()
    for b in range(batch):
        pk, ks, kz, kd = okivi.quantize_keys(f[b:b + 1], kstart[b], kstop[b], bits, group)
        g0, g1 = kstart[b] // group, kstop[b] // group
        np.testing.assert_array_equal(store.key_codes[b, :, kstart[b]:kstop[b]].cpu().numpy(), pk[0])
        np.testing.assert_array_equal(store.key_scale[b, :, g0:g1].cpu().numpy(), ks[0].astype(np.float16))
        np.testing.assert_array_equal(store.key_zero[b, :, g0:g1].cpu().numpy(), kz[0].astype(np.float16))
        if not ring:
            got = src_k[b, :, kstart[b]:kstop[b]].cpu()
            assert torch.equal(got, torch.from_numpy(kd[0]).to(dtype))
            assert torch.equal(src_k[b, :, kstop[b]:].cpu(), data[b, :, kstop[b]:])  # untouched
            pv, vs, vz, vd = okivi.quantize_values(f[b:b + 1], vstart[b], vstop[b], bits, group)
            np.testing.assert_array_equal(store.value_codes[b, :, vstart[b]:vstop[b]].cpu().numpy(), pv[0])
            np.testing.assert_array_equal(store.value_scale[b, :, vstart[b]:vstop[b]].cpu().numpy(),
                                          vs[0].astype(np.float16))
            np.testing.assert_array_equal(store.value_zero[b, :, vstart[b]:vstop[b]].cpu().numpy(),
                                          vz[0].astype(np.float16))
            assert store.value_scale.shape[3] == d // vg
            assert torch.equal(src_v[b, :, vstart[b]:vstop[b]].cpu(), torch.from_numpy(vd[0]).to(dtype))
            assert torch.equal(src_v[b, :, :vstart[b]].cpu(), data[b, :, :vstart[b]])


def test_pack_quantize_flags_scales_beyond_fp16() -> None:
    from economize_amd.kivi_packed import KIVIPackedStore

    data = torch.zeros(1, 1, 32, 64)
    data[0, 0, 0, 5] = 2e6  # a key group whose scale (2e6 / 3) lies beyond fp16
    store = KIVIPackedStore(1, 1, 32, 64, 64, 2, 32, "cuda")
    rows = lambda x: torch.tensor([x], dtype=torch.int32, device="cuda")  # noqa: E731
    store.quantize(data.cuda(), "k", rows(0), rows(32), 32)
    assert int(store.overflow.item()) == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("ring", [0, 40])
def test_dense_view_of_the_record(dtype, ring) -> None:
    """eco_kivi_packed_gather: the codes dequantized below each row's counts (equal to what the quantizer wrote back),
    the full-precision entries above them, from the buffer itself or from a ring at s % ring."""
    from economize_amd.kivi_packed import KIVIPackedStore

    batch, heads, slots, d, group, bits = 2, 2, 96, 48, 16, 4
    gen = torch.Generator().manual_seed(11)
    data = (torch.randn(batch, heads, slots, d, generator=gen) * 2).to(dtype)
    store = KIVIPackedStore(batch, heads, slots, d, d, bits, group, "cuda")
    written = data.clone().cuda()
    kq, vq = [64, 32], [70, 10]
    rows = lambda x: torch.tensor(x, dtype=torch.int32, device="cuda")  # noqa: E731
    keys_back, values_back = written.clone(), written.clone()
    store.quantize(keys_back, "k", rows([0, 0]), rows(kq), 64, write_back=True)
    store.quantize(values_back, "v", rows([0, 0]), rows(vq), 70, write_back=True)
    store.keys_quantized.copy_(rows(kq))
    store.values_quantized.copy_(rows(vq))
    if ring:
        src = torch.full((batch, heads, ring + 1, d), float("nan"), dtype=dtype, device="cuda")
        for s in range(slots - ring, slots):
            src[:, :, s % ring] = written[:, :, s]
        length = slots
        lows = [slots - ring] * batch
    else:
        src, length, lows = written, slots, [0] * batch
    keys, values = store.materialize(src, src, ring, length)
    torch.cuda.synchronize()
    for b in range(batch):
        assert torch.equal(keys[b, :, :kq[b]], keys_back[b, :, :kq[b]])
        assert torch.equal(values[b, :, :vq[b]], values_back[b, :, :vq[b]])
        lo_k, lo_v = max(kq[b], lows[b]), max(vq[b], lows[b])
        assert torch.equal(keys[b, :, lo_k:], written[b, :, lo_k:])
        assert torch.equal(values[b, :, lo_v:], written[b, :, lo_v:])
