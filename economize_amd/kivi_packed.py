"""KIVI codes in the reference's dense layout, read by the attention kernel (attention/kivi.py:80-309).

:class:`KIVIPacked` is the reference's record of one layer's packed K/V: codes ``[B, Hkv, S, D * bits / 8]``
(channel ``d`` in byte ``d // (8 // bits)`` at bit ``(d % (8 // bits)) * bits``), fp16 key scales and zero points per
channel and group of ``key_group`` tokens, fp16 value scales and zero points per token and group of ``value_group``
channels, and the per-row counts of quantized keys and values. :func:`kivi_decode_attention` attends over it: the
first ``keys_quantized[b]`` keys and ``values_quantized[b]`` values of row ``b`` are dequantized from their codes in
the kernel (``code * scale + zero`` in fp32, rounded to the query's dtype), every later slot comes from the dense
buffers or, for a cache without them, from the rings. Any bits (2, 4, 8), group, head dim up to 512 and query dtype
(bf16, fp16, fp32) run; the result is bit-identical to :func:`~economize_amd.decode.decode_attention` over buffers
holding the dequantized values, since both are the same kernel with a different load.

(The paged KIVI cache of :mod:`economize_amd.kivi` is this build's own packed layout, read by its own kernels.)
"""

from __future__ import annotations

import math
from collections.abc import Callable
from dataclasses import dataclass

import torch

from . import _lib
from .decode import DOT_DTYPES, _channel_contiguous, _workspace, mask_operand, sinks_operand
from .errors import ConfigError

__all__ = ["KIVIPacked", "KIVIPackedStore", "kivi_decode_attention"]


@dataclass
class KIVIPacked:
    """Packed K/V of one layer (the ``"kivi"`` packed format; the reference's record, attention/kivi.py:80-132).

    Attributes:
        bits: Bits per code (2, 4 or 8).
        key_group: Tokens per key scale (per channel).
        value_group: Channels per value scale (per token); it divides the value head dim.
        key_codes: ``uint8`` ``[B, Hkv, S, D * bits / 8]``.
        key_scale: fp16 ``[B, Hkv, ceil(S / key_group), D]``; ``key_zero`` has its shape and strides.
        value_codes: ``uint8`` ``[B, Hkv, S, Dv * bits / 8]``.
        value_scale: fp16 ``[B, Hkv, S, Dv / value_group]``; ``value_zero`` has its shape and strides.
        keys_quantized: ``int32`` ``[B]`` on the device: row ``b``'s keys below it are read as codes.
        values_quantized: ``int32`` ``[B]``: likewise for values.
        key_ring / value_ring: For a cache with no dense buffers (``ring > 0``), the full-precision K/V ``[B, Hkv, W,
            D]`` (``W >= ring``) in the query's dtype, slot ``s`` at ``s % ring``; ``None`` when the dense buffers
            handed to attention hold every slot that is not packed.
        ring: Slots of the rings, 0 without them.
        materialize: For a cache without dense buffers, a function returning the layer's dense K/V (for attention
            paths that do not read codes); ``None`` when the buffers handed over are dense.
    """

    bits: int
    key_group: int
    value_group: int
    key_codes: torch.Tensor
    key_scale: torch.Tensor
    key_zero: torch.Tensor
    value_codes: torch.Tensor
    value_scale: torch.Tensor
    value_zero: torch.Tensor
    keys_quantized: torch.Tensor
    values_quantized: torch.Tensor
    key_ring: torch.Tensor | None = None
    value_ring: torch.Tensor | None = None
    ring: int = 0
    materialize: Callable[[], tuple[torch.Tensor, torch.Tensor]] | None = None
    format: str = "kivi"

    def attend(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
               scale: float, softcap: float | None = None, sinks: torch.Tensor | None = None) -> torch.Tensor:
        return kivi_decode_attention(query, key, value, mask, scale, self, softcap=softcap, sinks=sinks)


def _layout(name: str, tensor: torch.Tensor, shape: tuple[int, ...], dtype: torch.dtype) -> None:
    """Refuses a tensor of another shape or dtype, or with a strided last axis."""
    if tuple(tensor.shape) != shape or tensor.dtype != dtype:
        raise ConfigError(f"KIVI {name}: got {tuple(tensor.shape)} {tensor.dtype}, the layout needs {shape} {dtype}")
    if tensor.stride(-1) != 1:
        raise ConfigError(f"KIVI {name}: the last axis must be contiguous")


def _aligned(tensor: torch.Tensor, nbytes: int) -> torch.Tensor:
    """``tensor``, or a contiguous copy when its base or strides are not multiples of ``nbytes`` (the kernel's
    chunk loads)."""
    es = tensor.element_size()
    if tensor.data_ptr() % nbytes == 0 and all((s * es) % nbytes == 0 for s in tensor.stride()[:-1]):
        return tensor
    return tensor.contiguous()


def kivi_decode_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
                          scale: float, packed: KIVIPacked, softcap: float | None = None,
                          sinks: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention over a cache whose oldest entries are KIVI codes (attention/kivi.py:199-309).

    Args:
        query: ``[B, Hq, Q, D]``, bf16, fp16 or fp32 (any strides).
        key: Dense ``[B, Hkv, S, D]`` in the query's dtype, read at slots ``>= packed.keys_quantized[b]`` only; with
            ``packed.ring`` only its shape is used (the full-precision keys come from ``packed.key_ring``).
        value: Dense ``[B, Hkv, S, Dv]``, likewise.
        mask: Boolean ``[B, 1 or Hq, Q or 1, S]`` or ``None``.
        scale: Multiplier of the scores.
        packed: The codes, scales, zero points and counts (:class:`KIVIPacked`).
        softcap: Optional tanh soft cap of the scaled scores.
        sinks: Optional ``[Hq]`` attention-sink logits.
        out: Optional ``[B, Q, Hq, Dv]`` output buffer.

    Returns:
        ``[B, Q, Hq, Dv]`` in the query's dtype.
    """
    device = _lib.require_gpu(query, key, value)
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ConfigError("kivi_decode_attention takes [B, Hq, Q, D] queries and [B, Hkv, S, D] keys and values")
    batch, q_heads, queries, head_dim = query.shape
    _, kv_heads, keys, _ = key.shape
    head_dv = value.shape[-1]
    ring = int(packed.ring)
    if ring:
        if packed.key_ring is None or packed.value_ring is None:
            raise ConfigError("KIVI packed K/V with ring > 0 needs key_ring and value_ring")
        if packed.key_ring.shape[2] < ring or packed.value_ring.shape[2] < ring:
            raise ConfigError(f"the KIVI rings hold {packed.key_ring.shape[2]} / {packed.value_ring.shape[2]} slots, "
                              f"fewer than ring = {ring}")
        dense_k, dense_v = packed.key_ring, packed.value_ring
    else:
        dense_k, dense_v = key, value
    if q_heads % kv_heads:
        raise ConfigError(f"{q_heads} query heads are not a multiple of {kv_heads} KV heads")
    if query.dtype not in DOT_DTYPES or dense_k.dtype != query.dtype or dense_v.dtype != query.dtype:
        raise ConfigError(f"kivi_decode_attention takes full-precision K/V in the query's dtype ({query.dtype}), "
                          f"got {dense_k.dtype} / {dense_v.dtype}")
    if dense_k.shape[:2] != (batch, kv_heads) or dense_v.shape[:2] != (batch, kv_heads) or \
            dense_k.shape[3] != head_dim or dense_v.shape[3] != head_dv or value.shape[:3] != key.shape[:3]:
        raise ConfigError(f"K {tuple(dense_k.shape)} / V {tuple(dense_v.shape)} do not match the query "
                          f"{tuple(query.shape)}")
    bits, kg, vg = int(packed.bits), int(packed.key_group), int(packed.value_group)
    if bits not in (2, 4, 8) or kg <= 0 or vg <= 0 or head_dim % (8 // bits) or head_dv % (8 // bits) or head_dv % vg:
        raise ConfigError(f"the KIVI layout bits={bits}, groups {kg} / {vg} does not fit head dims {head_dim} / "
                          f"{head_dv}")
    per_byte = 8 // bits
    rows = (batch, kv_heads)
    _layout("key_codes", packed.key_codes, (*rows, keys, head_dim // per_byte), torch.uint8)
    _layout("key_scale", packed.key_scale, (*rows, -(-keys // kg), head_dim), torch.float16)
    _layout("key_zero", packed.key_zero, (*rows, -(-keys // kg), head_dim), torch.float16)
    _layout("value_codes", packed.value_codes, (*rows, keys, head_dv // per_byte), torch.uint8)
    _layout("value_scale", packed.value_scale, (*rows, keys, head_dv // vg), torch.float16)
    _layout("value_zero", packed.value_zero, (*rows, keys, head_dv // vg), torch.float16)
    if packed.key_zero.stride() != packed.key_scale.stride() or \
            packed.value_zero.stride() != packed.value_scale.stride():
        raise ConfigError("KIVI zero points must share their scales' layout")
    for name in ("keys_quantized", "values_quantized"):
        counts = getattr(packed, name)
        if counts.shape != (batch,) or counts.dtype != torch.int32 or counts.device != device:
            raise ConfigError(f"KIVI {name} must be int32 [{batch}] on {device}")
    m, mask_strides = mask_operand(mask, keys)
    sinks = sinks_operand(sinks, q_heads)
    if out is not None and (out.shape != (batch, queries, q_heads, head_dv) or out.dtype != query.dtype or
                            out.stride(-1) != 1):
        raise ConfigError("out must be [B, Q, Hq, Dv] in the query's dtype with a contiguous last axis")
    if keys == 0:
        return torch.zeros(batch, queries, q_heads, head_dv, dtype=query.dtype, device=device) if out is None \
            else out.zero_()
    query, dense_k, dense_v = (_channel_contiguous(x) for x in (query, dense_k, dense_v))
    chunk = 16 // query.element_size()  # elements of the kernel's 16-byte chunks
    nb = chunk * bits // 8
    kc, vc = _aligned(packed.key_codes, nb), _aligned(packed.value_codes, nb)
    ks, kz = _aligned(packed.key_scale, 2 * chunk), _aligned(packed.key_zero, 2 * chunk)
    if ks.stride() != kz.stride():
        ks, kz = ks.contiguous(), kz.contiguous()
    vs, vz = packed.value_scale, packed.value_zero
    if out is None:
        out = torch.empty(batch, queries, q_heads, head_dv, dtype=query.dtype, device=device)
    need = int(_lib.lib().eco_decode_workspace_size(batch, queries, q_heads, kv_heads, keys, head_dim, head_dv))
    if need == 0:
        raise ConfigError(f"kivi_decode_attention supports head dims up to 512, got {head_dim} / {head_dv}")
    ws = _workspace(need, device, batch, queries, q_heads, kv_heads)
    _lib.call(
        "eco_kivi_packed_decode", query.data_ptr(), _lib.fmt(query.dtype), query.stride(0), query.stride(1),
        query.stride(2), dense_k.data_ptr(), dense_v.data_ptr(), dense_k.stride(0), dense_k.stride(1),
        dense_k.stride(2), dense_v.stride(0), dense_v.stride(1), dense_v.stride(2), ring,
        kc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), ks.data_ptr(), kz.data_ptr(), ks.stride(0),
        ks.stride(1), ks.stride(2), vc.data_ptr(), vc.stride(0), vc.stride(1), vc.stride(2), vs.data_ptr(),
        vz.data_ptr(), vs.stride(0), vs.stride(1), vs.stride(2), packed.keys_quantized.data_ptr(),
        packed.values_quantized.data_ptr(), bits, kg, vg, _lib.ptr(m), *mask_strides, _lib.ptr(sinks),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), batch, queries, q_heads, kv_heads, keys,
        head_dim, head_dv, float(scale if scale is not None else 1 / math.sqrt(head_dim)), float(softcap or 0.0),
        ws.data_ptr(), ws.numel(), _lib.stream_of(device),
    )
    return out


class KIVIPackedStore:
    """The codes, fp16 scales and zero points of one layer in the :class:`KIVIPacked` layout, for ``slots`` slots
    per row (the reference's ``_LayerStore``, techniques/kv_kivi_fused/fused.py:58-78), with the rows' quantized
    counts on the device and an overflow flag (a scale or zero point beyond fp16).

    Args:
        batch, heads, slots: Rows, KV heads and slots per row.
        head_dim, value_dim: Channels of keys and values (each packing into whole bytes at ``bits``).
        bits: 2, 4 or 8.
        group: Tokens per key group; channels per value group (the whole value head when it does not divide it,
            ``value_group`` of techniques/kv_quant/kivi.py:143-154).
    """

    def __init__(self, batch: int, heads: int, slots: int, head_dim: int, value_dim: int, bits: int, group: int,
                 device: torch.device) -> None:
        if bits not in (2, 4, 8):
            raise ConfigError(f"KIVI codes have 2, 4 or 8 bits, not {bits}")
        per_byte = 8 // bits
        for name, d in (("key", head_dim), ("value", value_dim)):
            if d % per_byte:
                raise ConfigError(f"the {name} head dim {d} does not pack into whole bytes at {bits} bits")
        self.bits, self.key_group = bits, group
        self.value_group = group if value_dim % group == 0 else value_dim
        self.slots = slots
        u8, f16 = torch.uint8, torch.float16
        self.key_codes = torch.zeros(batch, heads, slots, head_dim // per_byte, dtype=u8, device=device)
        self.key_scale = torch.zeros(batch, heads, -(-slots // group), head_dim, dtype=f16, device=device)
        self.key_zero = torch.zeros_like(self.key_scale)
        self.value_codes = torch.zeros(batch, heads, slots, value_dim // per_byte, dtype=u8, device=device)
        self.value_scale = torch.zeros(batch, heads, slots, value_dim // self.value_group, dtype=f16, device=device)
        self.value_zero = torch.zeros_like(self.value_scale)
        self.keys_quantized = torch.zeros(batch, dtype=torch.int32, device=device)
        self.values_quantized = torch.zeros(batch, dtype=torch.int32, device=device)
        self.overflow = torch.zeros(1, dtype=torch.int32, device=device)

    def quantize(self, source: torch.Tensor, kind: str, start: torch.Tensor, stop: torch.Tensor, max_tokens: int,
                 write_back: bool = False, ring: int = 0) -> None:
        """Quantize slots ``[start[b], stop[b])`` of every row of ``source`` ``[B, H, *, D]`` (bf16, fp16 or fp32,
        slot ``s`` at ``s % ring`` with a ring) into the record: ``kind`` ``"k"`` per channel over key groups (start
        and stop multiples of the group), ``"v"`` per token over value groups. ``write_back`` replaces the source's
        elements by their dequantized values (the dense buffers of the reference's fused cache). ``max_tokens``
        bounds ``stop - start`` over the rows."""
        if kind not in ("k", "v"):
            raise ConfigError(f"kind must be 'k' or 'v', not {kind!r}")
        if source.dim() != 4 or source.stride(-1) != 1:
            raise ConfigError("the source must be [B, H, slots, D] with a contiguous last axis")
        codes = self.key_codes if kind == "k" else self.value_codes
        scale, zero = (self.key_scale, self.key_zero) if kind == "k" else (self.value_scale, self.value_zero)
        group = self.key_group if kind == "k" else self.value_group
        batch, heads, _, dim = source.shape
        device = _lib.require_gpu(source, start, stop)
        start = start.to(torch.int32).contiguous()
        stop = stop.to(torch.int32).contiguous()
        _lib.call(
            "eco_kivi_pack_quantize", 0 if kind == "k" else 1, source.data_ptr(), _lib.fmt(source.dtype),
            source.stride(0), source.stride(1), source.stride(2), int(ring), int(write_back), codes.data_ptr(),
            codes.stride(0), codes.stride(1), codes.stride(2), scale.data_ptr(), zero.data_ptr(), scale.stride(0),
            scale.stride(1), scale.stride(2), start.data_ptr(), stop.data_ptr(), batch, heads, self.slots, dim,
            self.bits, group, int(max_tokens), self.overflow.data_ptr(), _lib.stream_of(device),
        )

    def record(self, length: int, key_ring: torch.Tensor | None = None, value_ring: torch.Tensor | None = None,
               ring: int = 0, materialize=None) -> KIVIPacked:
        """The :class:`KIVIPacked` view of the first ``length`` slots (views of the store, no copy)."""
        g = self.key_group
        return KIVIPacked(
            bits=self.bits, key_group=g, value_group=self.value_group,
            key_codes=self.key_codes[:, :, :length], key_scale=self.key_scale[:, :, : -(-length // g)],
            key_zero=self.key_zero[:, :, : -(-length // g)], value_codes=self.value_codes[:, :, :length],
            value_scale=self.value_scale[:, :, :length], value_zero=self.value_zero[:, :, :length],
            keys_quantized=self.keys_quantized, values_quantized=self.values_quantized, key_ring=key_ring,
            value_ring=value_ring, ring=ring, materialize=materialize,
        )

    def materialize(self, key_ring: torch.Tensor, value_ring: torch.Tensor, ring: int, length: int
                    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Fresh dense K/V ``[B, H, length, D]`` in the rings' dtype: the codes dequantized below the quantized
        counts, the rings (slot ``s`` at ``s % ring``; the slot itself with ``ring`` 0) above them
        (PackedKIVICache._dense, techniques/kv_quant/packed.py:300-320)."""
        device = _lib.require_gpu(key_ring, value_ring)
        out = []
        for kind, src, codes, scale, zero, counts, group in (
                (0, key_ring, self.key_codes, self.key_scale, self.key_zero, self.keys_quantized, self.key_group),
                (1, value_ring, self.value_codes, self.value_scale, self.value_zero, self.values_quantized,
                 self.value_group)):
            batch, heads, _, dim = src.shape
            dense = torch.empty(batch, heads, length, dim, dtype=src.dtype, device=device)
            if src.stride(-1) != 1:
                raise ConfigError("the rings need a contiguous last axis")
            out.append(dense)
            if length == 0:
                continue
            _lib.call(
                "eco_kivi_packed_gather", kind, codes.data_ptr(), codes.stride(0), codes.stride(1), codes.stride(2),
                scale.data_ptr(), zero.data_ptr(), scale.stride(0), scale.stride(1), scale.stride(2),
                counts.data_ptr(), src.data_ptr(), src.stride(0), src.stride(1), src.stride(2), int(ring),
                dense.data_ptr(), _lib.fmt(src.dtype), dense.stride(0), dense.stride(1), dense.stride(2), batch,
                heads, int(length), dim, self.bits, group, _lib.stream_of(device),
            )
        return out[0], out[1]
