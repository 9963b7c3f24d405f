"""Bit-level float helpers of the oracle: bf16 and fp16 rounding in numpy.

numpy has no bfloat16, so bf16 tensors are carried as their ``uint16`` bit patterns. Rounding float32 to bf16 is
round-to-nearest-even on the bit pattern, which is what ``torch.Tensor.to(torch.bfloat16)`` does on the CPU (the
reference casts with it everywhere, e.g. ``fp8_decode``'s ``.to(out)`` at techniques/kv_quant/fp8.py:92).

Pinned by: ``tests/test_oracle_fp8.py::test_bf16_and_fp16_rounding_match_torch`` compares the widening of every bf16
bit pattern, and the rounding of 2^20 random float32 values, exact round-half ties and special values, against
torch's own CPU casts.
"""

from __future__ import annotations

import numpy as np

__all__ = ["bf16_bits_to_f32", "f32_to_bf16_bits", "round_bf16", "round_fp16"]


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (``uint16``), round to nearest even, NaN kept quiet."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (``uint16``) -> float32 (exact)."""
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to bf16 precision, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_fp16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to fp16 (round to nearest even; overflow to inf), returned as float32."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
