"""Pins the oracle's KIVI quantizer, packing and schedule with hand-computed values, the reference's closed-form tests
(tests/techniques/test_kv_quant.py:72-118, 343-360) and torch's CPU arithmetic (the operators the reference's
``quantize`` runs, techniques/kv_quant/kivi.py:121-132)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kivi


def test_hand_computed_codes() -> None:
    codes, scale, low = kivi.quantize(np.float32([[0.0, 1.0, 2.0, 3.0]]), 2, axis=-1)
    assert codes.tolist() == [[0, 1, 2, 3]] and scale.item() == 1.0 and low.item() == 0.0
    # 0.5 / 1 rounds half to even (0); 2.5 would round to 2
    codes, _, _ = kivi.quantize(np.float32([[0.0, 0.5, 2.5, 3.0]]), 2, axis=-1)
    assert codes.tolist() == [[0, 0, 2, 3]]
    # scale 7 / 15 rounds to fp16 (0.46655273...), low exact
    codes, scale, low = kivi.quantize(np.float32([[-2.0, 5.0]]), 4, axis=-1)
    assert scale.item() == np.float32(np.float16(np.float32(7.0) / np.float32(15.0))) and low.item() == -2.0
    assert codes.tolist() == [[0, 15]]


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_levels_and_error_bound(bits: int) -> None:
    x = np.random.default_rng(0).standard_normal((3, 5, 64)).astype(np.float32)
    q = kivi.fake_quantize(x, bits, axis=-1)
    for row in q.reshape(-1, 64):
        assert np.unique(row).size <= 2**bits
    step = (x.max(-1, keepdims=True) - x.min(-1, keepdims=True)) / (2**bits - 1)
    assert (np.abs(q - x) <= step / 2 + 1e-3).all()


def test_constant_group_is_exact() -> None:
    x = np.full((2, 8), 0.25, np.float32)
    assert np.array_equal(kivi.fake_quantize(x, 2, axis=-1), x)


def test_matches_torch_cpu_arithmetic() -> None:
    """The reference's own closed form (test_kv_quant.py:353-359), evaluated with torch's CPU operators."""
    x = np.random.default_rng(2).standard_normal((64, 32)).astype(np.float32) * 7
    t = torch.from_numpy(x)
    low, high = t.amin(-1, keepdim=True), t.amax(-1, keepdim=True)
    for bits in (2, 4, 8):
        levels = 2**bits - 1
        scale, zero = ((high - low) / levels).half().float(), low.half().float()
        codes = ((t - zero) / torch.where(scale > 0, scale, torch.ones_like(scale))).round().clamp(0, levels)
        c, s, z = kivi.quantize(x, bits, axis=-1)
        assert np.array_equal(c, codes.numpy()) and np.array_equal(s, scale.numpy()) and np.array_equal(z, zero.numpy())
        assert np.array_equal(kivi.fake_quantize(x, bits, axis=-1), (codes * scale + zero).numpy())


def test_official_kivi_order_of_operations_agrees() -> None:
    """The official quantizer clamps before rounding (test_kv_quant_reference.py:33-43 describes it); on the
    level grid both orders give the same codes."""
    x = np.random.default_rng(3).standard_normal((16, 4, 32)).astype(np.float32)
    for bits in (2, 4):
        c, s, z = kivi.quantize(x, bits, axis=-1)
        safe = np.where(s > 0, s, 1).astype(np.float32)
        other = np.rint(np.clip(((x - z) / safe).astype(np.float32), 0, 2**bits - 1))
        assert np.array_equal(c, other)


def test_beyond_fp16_stays_finite() -> None:
    x = (np.random.default_rng(0).standard_normal((4, 64)) * 3e5).astype(np.float32)
    x[0, 0] = 1e6
    q = kivi.fake_quantize(x, 4, axis=-1)
    assert np.isfinite(q).all()
    _, scale, _ = kivi.quantize(x, 4, axis=-1)
    assert (np.abs(scale) > kivi.FP16_MAX).any()  # kept in fp32


def test_pack_bit_positions_and_round_trip() -> None:
    assert kivi.pack_codes(np.array([[1, 2, 3, 0]]), 2).tolist() == [[1 | 2 << 2 | 3 << 4]]
    assert kivi.pack_codes(np.array([[0xA, 0x5]]), 4).tolist() == [[0x5A]]
    rng = np.random.default_rng(4)
    for bits in (2, 4, 8):
        c = rng.integers(0, 2**bits, (3, 5, 64))
        assert np.array_equal(kivi.unpack_codes(kivi.pack_codes(c, bits), bits), c)


def test_schedule_and_bytes() -> None:
    assert kivi.schedule(8191, 128) == (8064, 8063)
    assert kivi.schedule(100, 128) == (0, 0)
    assert kivi.schedule(256, 128) == (256, 128)
    # the reference's example (test_kv_quant.py:95-104): bits 2, g 4, 2 heads, dim 16, fp32
    keys = 8 * 2 * 16 / 4 + 2 * 2 * 16 * 4
    values = 2 * 2 * 16 / 4 + 2 * 2 * (16 // 4) * 4
    assert kivi.kivi_bytes(10, 8, 2, 2, 16, 4, 2, 4) == keys + values + (2 + 8) * 2 * 16 * 4


def test_key_and_value_layouts() -> None:
    rng = np.random.default_rng(5)
    k = rng.standard_normal((2, 3, 96, 64)).astype(np.float32)
    packed, scale, zero, dense = kivi.quantize_keys(k, 32, 96, 4, 32)
    assert packed.shape == (2, 3, 64, 32) and scale.shape == (2, 3, 2, 64) and dense.shape == (2, 3, 64, 64)
    deq = kivi.dequantize(packed, scale, zero, 4, "key", 32, out="f32")
    assert np.array_equal(deq, dense)
    packed, scale, zero, dense = kivi.quantize_values(k, 0, 40, 2, 32)
    assert packed.shape == (2, 3, 40, 16) and scale.shape == (2, 3, 40, 2)
    assert np.array_equal(kivi.dequantize(packed, scale, zero, 2, "value", 32, out="f32"), dense)
