"""KIVI's cell layout on vLLM's paged cache (oracle).

Restates backends/vllm/kivi/layout.py:133-291 of the reference. One cell per (page, KV head, token)::

    [ K: D elements | V: D elements | value scales: nvg fp16 | value zeros: nvg fp16 |
      key aux: ka fp16 | key codes: D/pb bytes | value codes: D/pb bytes | key flag | value flag ]  (16-byte aligned)

* values per token over groups of ``vg`` channels (``vg = g`` when it divides ``D``, else ``D``): the cell holds its
  own ``nvg = D / vg`` scales and zero points;
* keys per channel over groups of ``g`` tokens: the group's ``2D`` fp16 values (``D`` scales, then ``D`` zero points)
  spread over its cells, ``ka = ceil(2D / g)`` per cell, entry ``e`` in the cell of token ``s0 + e // ka`` at aux
  slot ``e % ka``;
* codes packed along the channel axis, ``pb = 8 / bits`` per byte, channel ``j * pb + i`` at bits ``i * bits``;
* flags: 0 full precision, 1 quantized and packed, 2 a scale or zero point beyond fp16 (codes unused); a quantized
  cell's dense entry holds the dequantized value.

Pinned by (``tests/test_oracle_vllm_cells.py``): ``read_cells(write_cells(...))`` equals :func:`oracle.kivi.
fake_quantize` of the same groups (the reference's test_vllm_kivi.py:120-141 check), the byte position of single
codes and of single aux entries against the layout's stated formulas, the offsets against the layout's closed
forms, and untouched full-precision cells.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .kivi import quantize

__all__ = ["FLAG_DENSE", "FLAG_OVERFLOW", "FLAG_PACKED", "CellLayout", "cell_layout", "read_cells", "write_cells"]

FLAG_DENSE, FLAG_PACKED, FLAG_OVERFLOW = 0, 1, 2
_FP16_MAX = np.float32(65504.0)


@dataclass(frozen=True)
class CellLayout:
    """Byte offsets inside one cell (layout.py:133-193)."""

    head_size: int
    element_size: int
    bits: int
    group_size: int
    value_group: int
    key_aux: int

    @property
    def value_groups(self) -> int:
        return self.head_size // self.value_group

    @property
    def code_bytes(self) -> int:
        return self.head_size // (8 // self.bits)

    @property
    def off_v(self) -> int:
        return self.head_size * self.element_size

    @property
    def off_vs(self) -> int:
        return 2 * self.head_size * self.element_size

    @property
    def off_vz(self) -> int:
        return self.off_vs + 2 * self.value_groups

    @property
    def off_ka(self) -> int:
        return self.off_vz + 2 * self.value_groups

    @property
    def off_kc(self) -> int:
        return self.off_ka + 2 * self.key_aux

    @property
    def off_vc(self) -> int:
        return self.off_kc + self.code_bytes

    @property
    def off_flag(self) -> int:
        return self.off_vc + self.code_bytes

    @property
    def size(self) -> int:
        return -(-(self.off_flag + 2) // 16) * 16


def cell_layout(head_size: int, element_size: int, bits: int, group_size: int) -> CellLayout:
    """The cell of ``head_size`` channels of ``element_size`` bytes (layout.py:196-213)."""
    value_group = group_size if head_size % group_size == 0 else head_size
    key_aux = -(-2 * head_size // group_size)
    return CellLayout(head_size, element_size, bits, group_size, value_group, key_aux)


def _pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """Codes ``[..., D]`` packed along the last axis, ``8 / bits`` per byte, channel ``j pb + i`` at bit ``i bits``."""
    pb = 8 // bits
    c = codes.astype(np.int64).reshape(*codes.shape[:-1], codes.shape[-1] // pb, pb)
    return (c << (np.arange(pb) * bits)).sum(-1).astype(np.uint8)


def _to_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values rounded to the cache dtype, as that dtype's raw bytes ``[..., D * es]``."""
    from .numerics import f32_to_bf16_bits

    if dtype == "bf16":
        return f32_to_bf16_bits(x).view(np.uint8).reshape(*x.shape[:-1], -1)
    if dtype == "f16":
        return x.astype(np.float16).view(np.uint8).reshape(*x.shape[:-1], -1)
    return x.astype(np.float32).view(np.uint8).reshape(*x.shape[:-1], -1)


def write_cells(keys: np.ndarray, values: np.ndarray, keys_quantized: int, values_quantized: int, layout: CellLayout,
                dtype: str) -> np.ndarray:
    """uint8 ``[H, S, layout.size]`` cells of one sequence whose first ``keys_quantized`` keys (whole groups) and
    ``values_quantized`` values are quantized, from its K/V ``[H, S, D]`` (float32 holding values of ``dtype``:
    ``"bf16"``, ``"f16"`` or ``"f32"``) (layout.py:222-256)."""
    heads, tokens, dim = keys.shape
    g, vg, bits = layout.group_size, layout.value_group, layout.bits
    if keys_quantized % g:
        raise ValueError(f"{keys_quantized} quantized keys are not whole groups of {g}")
    cells = np.zeros((heads, tokens, layout.size), np.uint8)
    dense_k = np.array(keys, np.float32, copy=True)
    dense_v = np.array(values, np.float32, copy=True)
    if keys_quantized:
        block = dense_k[:, :keys_quantized].reshape(heads, keys_quantized // g, g, dim)
        codes, scale, low = quantize(block, bits, axis=2)
        dense_k[:, :keys_quantized] = ((codes * scale).astype(np.float32) + low).reshape(heads, -1, dim)
        cells[:, :keys_quantized, layout.off_kc:layout.off_vc] = _pack(codes.reshape(heads, -1, dim), bits)
        over = ((np.abs(scale) > _FP16_MAX) | (np.abs(low) > _FP16_MAX)).any(axis=-1)  # [H, G, 1]
        flags = np.where(over, FLAG_OVERFLOW, FLAG_PACKED)
        cells[:, :keys_quantized, layout.off_flag] = np.broadcast_to(flags, (heads, keys_quantized // g, g)) \
            .reshape(heads, -1)
        with np.errstate(over="ignore"):  # a scale beyond fp16 stores inf (its flag says so)
            aux = np.concatenate([scale[:, :, 0], low[:, :, 0]], axis=-1).astype(np.float16)  # [H, G, 2D]
        pad = g * layout.key_aux - 2 * dim
        aux = np.concatenate([aux, np.zeros((heads, aux.shape[1], pad), np.float16)], axis=-1)
        cells[:, :keys_quantized, layout.off_ka:layout.off_kc] = aux.reshape(heads, -1, layout.key_aux) \
            .view(np.uint8).reshape(heads, keys_quantized, -1)
    if values_quantized:
        block = dense_v[:, :values_quantized].reshape(heads, values_quantized, dim // vg, vg)
        codes, scale, low = quantize(block, bits, axis=3)
        dense_v[:, :values_quantized] = ((codes * scale).astype(np.float32) + low).reshape(heads, -1, dim)
        cells[:, :values_quantized, layout.off_vc:layout.off_flag] = _pack(codes.reshape(heads, -1, dim), bits)
        over = ((np.abs(scale) > _FP16_MAX) | (np.abs(low) > _FP16_MAX)).reshape(heads, values_quantized, -1)
        cells[:, :values_quantized, layout.off_flag + 1] = np.where(over.any(-1), FLAG_OVERFLOW, FLAG_PACKED)
        with np.errstate(over="ignore"):
            cells[:, :values_quantized, layout.off_vs:layout.off_vz] = scale.reshape(heads, values_quantized, -1) \
                .astype(np.float16).view(np.uint8)
            cells[:, :values_quantized, layout.off_vz:layout.off_ka] = low.reshape(heads, values_quantized, -1) \
                .astype(np.float16).view(np.uint8)
    cells[:, :, :layout.off_v] = _to_dtype(dense_k, dtype)
    cells[:, :, layout.off_v:layout.off_vs] = _to_dtype(dense_v, dtype)
    return cells


def _from_dtype(raw: np.ndarray, dtype: str) -> np.ndarray:
    from .numerics import bf16_bits_to_f32

    if dtype == "bf16":
        return bf16_bits_to_f32(np.ascontiguousarray(raw).view(np.uint16))
    if dtype == "f16":
        return np.ascontiguousarray(raw).view(np.float16).astype(np.float32)
    return np.ascontiguousarray(raw).view(np.float32).copy()


def read_cells(cells: np.ndarray, layout: CellLayout, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """float32 K/V ``[H, S, D]`` the cells hold: dequantized codes where a flag is 1, dense entries elsewhere
    (layout.py:259-291)."""
    heads, tokens, _ = cells.shape
    dim, g, vg, bits = layout.head_size, layout.group_size, layout.value_group, layout.bits
    pb = 8 // bits
    keys = _from_dtype(cells[:, :, :layout.off_v], dtype)
    values = _from_dtype(cells[:, :, layout.off_v:layout.off_vs], dtype)

    def unpack(raw: np.ndarray) -> np.ndarray:
        shifts = np.arange(pb) * bits
        return ((raw.astype(np.int32)[..., None] >> shifts) & (2**bits - 1)).reshape(*raw.shape[:-1], dim) \
            .astype(np.float32)

    def rounded(x: np.ndarray) -> np.ndarray:
        return _from_dtype(_to_dtype(x, dtype), dtype)

    errors = np.seterr(over="ignore", invalid="ignore")  # an overflowed group's codes are not read

    groups = tokens // g
    if groups:
        aux = np.ascontiguousarray(cells[:, :groups * g, layout.off_ka:layout.off_kc]).view(np.float16)
        aux = aux.reshape(heads, groups, g * layout.key_aux)[..., :2 * dim].astype(np.float32)
        scale = np.repeat(aux[..., :dim], g, axis=1)
        zero = np.repeat(aux[..., dim:], g, axis=1)
        codes = unpack(cells[:, :groups * g, layout.off_kc:layout.off_vc])
        deq = rounded(((codes * scale).astype(np.float32) + zero).astype(np.float32))
        packed = cells[:, :groups * g, layout.off_flag] == FLAG_PACKED
        keys[:, :groups * g] = np.where(packed[..., None], deq, keys[:, :groups * g])
    vscale = np.ascontiguousarray(cells[:, :, layout.off_vs:layout.off_vz]).view(np.float16).astype(np.float32)
    vzero = np.ascontiguousarray(cells[:, :, layout.off_vz:layout.off_ka]).view(np.float16).astype(np.float32)
    codes = unpack(cells[:, :, layout.off_vc:layout.off_flag])
    deq = rounded(((codes * np.repeat(vscale, vg, axis=-1)).astype(np.float32) +
                   np.repeat(vzero, vg, axis=-1)).astype(np.float32))
    packed = cells[:, :, layout.off_flag + 1] == FLAG_PACKED
    values = np.where(packed[..., None], deq, values)
    np.seterr(**errors)
    return keys, values
