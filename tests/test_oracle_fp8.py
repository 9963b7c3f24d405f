"""Pins the oracle's fp8 encode/decode to torch's own CPU casts (the operators the reference's ``fp8_encode`` /
``fp8_decode`` call, techniques/kv_quant/fp8.py:81-92) and to closed-form byte values."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16, round_fp16

TORCH_FP8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _torch_encode(x: np.ndarray, fmt: str) -> np.ndarray:
    limit = torch.finfo(TORCH_FP8[fmt]).max
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).clamp(-limit, limit)
    return t.to(TORCH_FP8[fmt]).view(torch.uint8).numpy()


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_every_bf16_input_encodes_like_torch(fmt: str) -> None:
    x = bf16_bits_to_f32(np.arange(65536, dtype=np.uint16))
    x = x[np.isfinite(x)]
    limit = np.float32(fp8.FORMATS[fmt][3])
    assert np.array_equal(fp8.fp8_encode(x, fmt, None), _torch_encode(np.clip(x, -limit, limit), fmt))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_random_fp32_and_scaled_inputs_encode_like_torch(fmt: str) -> None:
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(1 << 20) * np.exp2(rng.integers(-20, 12, 1 << 20))).astype(np.float32)
    limit = np.float32(fp8.FORMATS[fmt][3])
    assert np.array_equal(fp8.fp8_encode(x, fmt, None), _torch_encode(np.clip(x, -limit, limit), fmt))
    scale = np.float32(0.0123)
    want = _torch_encode(np.clip((torch.from_numpy(x) / float(scale)).numpy(), -limit, limit), fmt)
    assert np.array_equal(fp8.fp8_encode(x, fmt, scale), want)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_decode_table_is_torchs(fmt: str) -> None:
    raw = torch.arange(256, dtype=torch.uint8)
    want = raw.view(TORCH_FP8[fmt]).float().numpy()
    got = fp8.decode_table(fmt)
    finite = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[finite], want[finite])


def test_closed_form_bytes() -> None:
    table = fp8.decode_table("e4m3")
    assert table[0x38] == 1.0 and table[0x7E] == 448.0 and table[0x01] == 2.0**-9 and table[0x08] == 2.0**-6
    assert np.isnan(table[0x7F]) and table[0xBE] == -1.75 * 2**0
    assert fp8.e4m3_encode(np.float32([1.0, 448.0, 2.0**-9, 1.0625, 1.1875]))[:5].tolist() == [0x38, 0x7E, 0x01,
                                                                                              0x38, 0x3A]


def test_saturation_after_the_clamp() -> None:
    big = np.float32([1e6, -1e6, 460.0, 449.0])
    assert fp8.fp8_encode(big, "e4m3", None).tolist() == [0x7E, 0xFE, 0x7E, 0x7E]


def test_decode_rounds_to_bf16() -> None:
    raw = np.arange(256, dtype=np.uint8)
    scale = np.float32(0.3)
    got = fp8.fp8_decode(raw, "e4m3", scale, "bf16")
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float() * 0.3
    want = t.to(torch.bfloat16).float().numpy()
    ok = np.isfinite(want)
    assert np.array_equal(got[ok], want[ok])


def test_scales_follow_the_reference_rules() -> None:
    x = np.float32([[[[1.0, -896.0], [0.0, 0.0]]]])  # [1, 1, 2, 2]
    assert fp8.token_scale(x, "e4m3")[0, 0, :, 0].tolist() == [2.0, np.float32(1e-12)]
    assert fp8.static_scales(np.float32([0.0, 896.0]), "e4m3").tolist() == [1.0, 2.0]
    heads = np.zeros((2, 3, 4, 8), np.float32)
    heads[1, 2, 3, 5] = -44.8
    assert np.allclose(fp8.head_scales(heads, "e4m3"), [1.0, 1.0, np.float32(44.8) / np.float32(448.0)])


def test_bf16_and_fp16_rounding_match_torch() -> None:
    """oracle.numerics against torch's CPU casts: every bf16 bit pattern widens as torch widens it, and 2^20 random
    float32 values plus exact round-half ties, infinities, NaN and fp16 overflow round as torch rounds them."""
    from oracle.numerics import bf16_bits_to_f32

    patterns = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    widened = torch.from_numpy(patterns.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(bf16_bits_to_f32(patterns).view(np.uint32), widened.view(np.uint32))
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(1 << 20) * np.exp2(rng.integers(-30, 30, 1 << 20))).astype(np.float32)
    # exact halfway points between neighbouring bf16 values (both parities) and special values
    base = rng.integers(0, 1 << 16, 4096).astype(np.uint32) << 16
    ties = (base | np.uint32(0x8000)).view(np.float32)
    special = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 65504.0, 65520.0, 1e6, -3.4e38], np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)], special])
    t = torch.from_numpy(x)
    assert np.array_equal(round_bf16(x), t.to(torch.bfloat16).float().numpy(), equal_nan=True)
    assert np.array_equal(f32_to_bf16_bits(x)[np.isfinite(x)],
                          t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)[np.isfinite(x)])
    assert np.array_equal(round_fp16(x), t.half().float().numpy(), equal_nan=True)
