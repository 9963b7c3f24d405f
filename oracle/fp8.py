"""FP8 KV encode/decode and scales (oracle).

Follows techniques/kv_quant/fp8.py of the reference:

* ``fp8_encode`` (fp8.py:81-86): ``x.float() / scale`` (IEEE division), clamped to the format's finite maximum, cast
  to the fp8 format with round-to-nearest-even, stored as bytes.
* ``fp8_decode`` (fp8.py:89-92): the byte's exact value times the scale, rounded to the output dtype.
* ``token_scale`` (fp8.py:95-97) and ``static_scales`` (fp8.py:130-133); ``head_scales`` applies the
  ``static_scales`` rule per KV head instead of per layer, the per-head mode of the fp8 paged path.

The byte <-> value maps are written from the OCP 8-bit float definitions (e4m3fn: bias 7, no infinities, 0x7F/0xFF
NaN, max 448; e5m2: bias 15, IEEE-like, max 57344).

Pinned by (``tests/test_oracle_fp8.py``): every bf16 bit pattern and 2^20 random float32 values encoded by torch's
own CPU ``Tensor.to(torch.float8_*)`` (the call the reference makes at fp8.py:86), the 256-byte decode table against
torch's ``view(fp8).float()`` (fp8.py:91) and the closed-form values of a few bytes (0x38 = 1.0, 0x7E = 448,
0x01 = 2^-9). End to end, ``tests/test_golden_reference.py`` decodes the reference's golden model with every K/V
through this round trip and gets the reference's own ``kv_fp8`` golden tokens (tests/golden/catalog.py:168-170).
"""

from __future__ import annotations

import numpy as np

from .numerics import f32_to_bf16_bits, round_bf16

__all__ = [
    "FORMATS",
    "decode_table",
    "e4m3_encode",
    "e5m2_encode",
    "fp8_decode",
    "fp8_encode",
    "head_scales",
    "static_scales",
    "token_scale",
]

#: Format name -> (exponent bits, mantissa bits, bias, finite maximum).
FORMATS = {"e4m3": (4, 3, 7, 448.0), "e5m2": (5, 2, 15, 57344.0)}


def _encode(x: np.ndarray, fmt: str) -> np.ndarray:
    """Round-to-nearest-even cast of float32 values inside the finite range to fp8 bytes."""
    ebits, mbits, bias, _ = FORMATS[fmt]
    a = np.asarray(x, dtype=np.float32)
    sign = np.signbit(a).astype(np.uint8) << 7
    mag = np.abs(a).astype(np.float64)
    min_normal = 2.0 ** (1 - bias)
    out = np.zeros(a.shape, dtype=np.uint8)
    sub = mag < min_normal
    # subnormals (and zero): multiples of 2^(1 - bias - mbits), rounded half to even
    m_sub = np.rint(mag[sub] / 2.0 ** (1 - bias - mbits)).astype(np.int64)  # 2^mbits rounds up to the min normal
    out[sub] = m_sub.astype(np.uint8)
    norm = ~sub
    if norm.any():
        mn = mag[norm]
        e = np.floor(np.log2(mn)).astype(np.int64)
        # guard against log2 rounding at exact powers of two
        e = np.where(2.0 ** e > mn, e - 1, e)
        e = np.where(2.0 ** (e + 1) <= mn, e + 1, e)
        q = np.rint(mn / 2.0 ** (e - mbits)).astype(np.int64)  # in [2^mbits, 2^(mbits+1)]
        carry = q == (1 << (mbits + 1))
        e = np.where(carry, e + 1, e)
        q = np.where(carry, 1 << mbits, q)
        code = ((e + bias) << mbits) | (q - (1 << mbits))
        out[norm] = code.astype(np.uint8)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, np.uint8((1 << (ebits + mbits)) - 1 if fmt == "e4m3" else 0x7F), out)
    return out | sign


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn bytes (values must already lie in [-448, 448])."""
    return _encode(x, "e4m3")


def e5m2_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e5m2 bytes (values must already lie in [-57344, 57344])."""
    return _encode(x, "e5m2")


def decode_table(fmt: str) -> np.ndarray:
    """float32 ``[256]``: the exact value of every byte of the format (NaN for its NaN codes)."""
    ebits, mbits, bias, _ = FORMATS[fmt]
    b = np.arange(256, dtype=np.int64)
    s = np.where(b >> 7, -1.0, 1.0)
    e = (b >> mbits) & ((1 << ebits) - 1)
    m = b & ((1 << mbits) - 1)
    sub = s * m * 2.0 ** (1 - bias - mbits)
    norm = s * (1.0 + m / float(1 << mbits)) * 2.0 ** (e - bias)
    val = np.where(e == 0, sub, norm)
    if fmt == "e4m3":
        val = np.where((e == 15) & (m == 7), np.nan, val)
    else:
        val = np.where(e == 31, np.where(m == 0, s * np.inf, np.nan), val)
    return val.astype(np.float32)


def fp8_encode(x: np.ndarray, fmt: str, scale: np.ndarray | float | None) -> np.ndarray:
    """``x / scale`` clamped to the format's maximum and cast to fp8 bytes (fp8.py:81-86).

    ``x`` is float32 (a bf16 input is widened exactly first); ``scale`` broadcasts against ``x`` (a scalar, a
    per-token ``[..., 1]`` or a per-head array) or is ``None``.
    """
    limit = np.float32(FORMATS[fmt][3])
    work = np.asarray(x, dtype=np.float32)
    if scale is not None:
        work = (work / np.asarray(scale, dtype=np.float32)).astype(np.float32)
    return _encode(np.clip(work, -limit, limit), fmt)


def fp8_decode(raw: np.ndarray, fmt: str, scale: np.ndarray | float | None, out: str = "bf16") -> np.ndarray:
    """The float32 values of ``out`` precision that ``raw`` decodes to (fp8.py:89-92): ``value * scale`` in fp32,
    then rounded to ``out`` (``"bf16"`` or ``"f32"``)."""
    work = decode_table(fmt)[np.asarray(raw, dtype=np.uint8)]
    if scale is not None:
        work = (work * np.asarray(scale, dtype=np.float32)).astype(np.float32)
    if out == "bf16":
        return round_bf16(work)
    if out == "f32":
        return work
    raise ValueError(out)


def token_scale(x: np.ndarray, fmt: str) -> np.ndarray:
    """Per-token, per-head scale ``[..., 1]``: absmax over the last axis / format max, at least 1e-12
    (fp8.py:95-97)."""
    amax = np.abs(np.asarray(x, dtype=np.float32)).max(axis=-1, keepdims=True)
    s = (amax / np.float32(FORMATS[fmt][3])).astype(np.float32)
    return np.maximum(s, np.float32(1e-12))


def static_scales(absmax: np.ndarray, fmt: str) -> np.ndarray:
    """absmax / format max, 1 where the absmax is 0 (fp8.py:130-133)."""
    s = (np.asarray(absmax, dtype=np.float32) / np.float32(FORMATS[fmt][3])).astype(np.float32)
    return np.where(s > 0, s, np.float32(1.0)).astype(np.float32)


def head_scales(x: np.ndarray, fmt: str) -> np.ndarray:
    """Per-KV-head scales of ``x`` ``[..., H, S, D]`` laid out ``[B, H, S, D]``: the ``static_scales`` rule over each
    head's absolute maximum (the per-head absmax scale of the fp8 paged path)."""
    a = np.abs(np.asarray(x, dtype=np.float32))
    amax = a.max(axis=tuple(i for i in range(a.ndim) if i != a.ndim - 3))
    return static_scales(amax, fmt)


def encode_bf16_input(x_bf16_bits: np.ndarray, fmt: str, scale) -> np.ndarray:
    """:func:`fp8_encode` of bf16 inputs given as bit patterns."""
    from .numerics import bf16_bits_to_f32

    return fp8_encode(bf16_bits_to_f32(x_bf16_bits), fmt, scale)

