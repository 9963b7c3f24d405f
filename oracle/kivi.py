"""KIVI quantization, packing, dequantization and schedule (oracle).

Follows the reference:

* ``quantize`` / ``fake_quantize`` / ``_fp16_rounded`` (techniques/kv_quant/kivi.py:110-140): fp32 min and max along
  the group axis; ``scale = fp16r((high - low) / levels)`` with IEEE division by the level count (the CPU semantics
  of ``tensor / int``); ``low = fp16r(low)``; ``codes = round_half_even((x - low) / safe)`` clamped to
  ``[0, levels]``, ``safe`` the scale or 1 where the scale is 0; ``fp16r`` keeps fp32 where ``|x| > 65504``.
* ``pack_codes`` / ``unpack_codes`` / ``dequantize`` (attention/kivi.py:38-76): channel ``d`` in byte
  ``d // (8 // bits)`` at bit ``(d % (8 // bits)) * bits``; ``dequantize`` is ``code * scale + zero`` in fp32
  (two roundings, no fused multiply-add) cast to the output dtype.
* the schedule of ``KIVICache._plan`` (techniques/kv_quant/kivi.py:230-243): with ``c`` committed tokens,
  ``(c // R) * R`` keys and ``max(0, c - R)`` values are quantized.
* ``kivi_bytes`` (techniques/kv_quant/kivi.py:163-175), the bytes of one layer's K and V.
* ``quantize_keys`` / ``quantize_values`` lay the results out as ``KIVIPacked`` holds them (attention/kivi.py:80-120):
  key scales ``[B, H, ceil(S / G), D]``, value scales ``[B, H, S, D / G]``, codes ``[B, H, S, D * bits / 8]``.

Pinned by (``tests/test_oracle_kivi.py``): the reference's closed-form tests (techniques/test_kv_quant.py:72-86,
343-360: level counts, error bound, constant groups exact, the fp16-rounded scale formula, finite beyond the fp16
range), a transcription-free restatement of the official KIVI quantizer's order of operations (clamp then round,
test_kv_quant_reference.py:33-43 describes it), pack/unpack identity and the bit positions of single codes, and the
``kivi_bytes`` example of test_kv_quant.py:95-104. End to end, ``tests/test_golden_reference.py`` decodes the
reference's golden model with :func:`schedule`, :func:`quantize_keys` and :func:`quantize_values` at 2 bits, groups
of 4 and residual 8, and gets the reference's own ``kv_kivi_2bit`` golden tokens (tests/golden/catalog.py:163-165).
"""

from __future__ import annotations

import numpy as np

from .numerics import round_bf16

__all__ = [
    "FP16_MAX",
    "dequantize",
    "fake_quantize",
    "fp16_rounded",
    "kivi_bytes",
    "pack_codes",
    "quantize",
    "quantize_keys",
    "quantize_values",
    "schedule",
    "unpack_codes",
]

FP16_MAX = np.float32(65504.0)


def fp16_rounded(x: np.ndarray) -> np.ndarray:
    """``x`` (fp32) rounded to fp16 where fp16 represents it, unchanged beyond 65504 (kivi.py:138-140)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        half = x.astype(np.float16).astype(np.float32)
    return np.where(np.abs(x) <= FP16_MAX, half, x).astype(np.float32)


def quantize(x: np.ndarray, bits: int, axis: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``(codes, scale, low)`` of KIVI's min-max quantization along ``axis`` (kivi.py:121-132); codes as float32,
    scale and low keep ``axis`` with size 1."""
    work = np.asarray(x, dtype=np.float32)
    low = work.min(axis=axis, keepdims=True)
    high = work.max(axis=axis, keepdims=True)
    levels = np.float32(2**bits - 1)
    scale = fp16_rounded(((high - low).astype(np.float32) / levels).astype(np.float32))
    low = fp16_rounded(low)
    safe = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    codes = np.clip(np.rint(((work - low).astype(np.float32) / safe).astype(np.float32)), 0, levels)
    return codes.astype(np.float32), scale, low


def fake_quantize(x: np.ndarray, bits: int, axis: int) -> np.ndarray:
    """``codes * scale + low`` in fp32 (kivi.py:110-118), before the cast to the cache dtype."""
    codes, scale, low = quantize(x, bits, axis)
    return ((codes * scale).astype(np.float32) + low).astype(np.float32)


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Integer codes ``[..., D]`` packed along the last axis into ``uint8`` ``[..., D * bits / 8]``
    (attention/kivi.py:38-45)."""
    per_byte = 8 // bits
    c = np.asarray(codes).astype(np.int64)
    if c.shape[-1] % per_byte:
        raise ValueError(f"{c.shape[-1]} channels do not pack into whole bytes at {bits} bits")
    grouped = c.reshape(*c.shape[:-1], c.shape[-1] // per_byte, per_byte)
    shifts = np.arange(per_byte, dtype=np.int64) * bits
    return (grouped << shifts).sum(-1).astype(np.uint8)


def unpack_codes(packed: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of :func:`pack_codes` (``int32`` codes, attention/kivi.py:48-53)."""
    per_byte = 8 // bits
    shifts = np.arange(per_byte, dtype=np.int32) * bits
    codes = (np.asarray(packed).astype(np.int32)[..., None] >> shifts) & (2**bits - 1)
    return codes.reshape(*packed.shape[:-1], packed.shape[-1] * per_byte)


def dequantize(codes_packed: np.ndarray, scale: np.ndarray, zero: np.ndarray, bits: int, axis: str, group: int,
               out: str = "bf16") -> np.ndarray:
    """Dense values of packed codes ``[B, H, S, D / per_byte]`` (attention/kivi.py:56-76): ``code * scale + zero``
    in fp32, rounded to ``out``. ``scale``/``zero`` are ``[B, H, ceil(S / G), D]`` for keys, ``[B, H, S, D / G]``
    for values (float32 holding fp16 values)."""
    c = unpack_codes(codes_packed, bits).astype(np.float32)
    s = np.asarray(scale, dtype=np.float32)
    z = np.asarray(zero, dtype=np.float32)
    if axis == "key":
        s = np.repeat(s, group, axis=2)[:, :, : c.shape[2]]
        z = np.repeat(z, group, axis=2)[:, :, : c.shape[2]]
    else:
        s = np.repeat(s, group, axis=3)
        z = np.repeat(z, group, axis=3)
    v = ((c * s).astype(np.float32) + z).astype(np.float32)
    return round_bf16(v) if out == "bf16" else v


def schedule(committed: int, residual: int) -> tuple[int, int]:
    """``(keys_quantized, values_quantized)`` once a row holds ``committed`` committed tokens (kivi.py:238)."""
    return (committed // residual) * residual, max(0, committed - residual)


def kivi_bytes(tokens, keys_quantized, values_quantized, heads: int, dim: int, element: int, bits: int,
               group: int, scale_bytes: int = 2):
    """Bytes of one layer's K and V (kivi.py:163-175)."""
    value_groups = dim // group if dim % group == 0 else 1
    per_bit = bits / 8
    pair = 2 * scale_bytes
    keys = keys_quantized * heads * dim * per_bit + (keys_quantized // group) * heads * dim * pair
    values = values_quantized * heads * dim * per_bit + values_quantized * heads * value_groups * pair
    full = ((tokens - keys_quantized) + (tokens - values_quantized)) * heads * dim * element
    return keys + values + full


def quantize_keys(keys: np.ndarray, start: int, stop: int, bits: int, group: int
                  ) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Key slots ``start:stop`` (multiples of ``group``) of ``keys`` ``[B, H, S, D]`` (float32 holding the cache's
    values) quantized per channel over groups of ``group`` tokens, as ``FusedKIVICache._quantize_block`` stores them
    (techniques/kv_kivi_fused/fused.py:152-160).

    Returns ``(packed codes [B, H, T, D*bits/8], scale [B, H, T/G, D], zero [B, H, T/G, D], dequantized fp32
    [B, H, T, D])`` for the ``T = stop - start`` slots.
    """
    block = np.asarray(keys[:, :, start:stop], dtype=np.float32)
    b, h, t, d = block.shape
    codes, scale, low = quantize(block.reshape(b, h, t // group, group, d), bits, axis=3)
    dense = ((codes * scale).astype(np.float32) + low).astype(np.float32).reshape(block.shape)
    packed = pack_codes(codes.reshape(block.shape).astype(np.int64), bits)
    return packed, scale.squeeze(3), low.squeeze(3), dense


def quantize_values(values: np.ndarray, start: int, stop: int, bits: int, group: int
                    ) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Value slots ``start:stop`` of ``values`` ``[B, H, S, D]`` quantized per token over groups of ``group``
    channels (techniques/kv_kivi_fused/fused.py:161-166; ``value_group`` of kivi.py:143-154 picks the whole head
    when ``group`` does not divide it).

    Returns ``(packed codes [B, H, T, D*bits/8], scale [B, H, T, D/G], zero [B, H, T, D/G], dequantized fp32)``.
    """
    block = np.asarray(values[:, :, start:stop], dtype=np.float32)
    b, h, t, d = block.shape
    g = group if d % group == 0 else d
    codes, scale, low = quantize(block.reshape(b, h, t, d // g, g), bits, axis=4)
    dense = ((codes * scale).astype(np.float32) + low).astype(np.float32).reshape(block.shape)
    packed = pack_codes(codes.reshape(block.shape).astype(np.int64), bits)
    return packed, scale.squeeze(4), low.squeeze(4), dense
