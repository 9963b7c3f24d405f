"""Decode attention over dense K/V buffers on the GPU: the reference's ``decode_attention`` (attention/decode.py:
252-324) on the HIP kernels of ``dense_attention.hip``.

It serves the caches that keep dense ``[B, Hkv, S, D]`` buffers, as the reference's model caches do (the fused fp8
cache hands its fp8 buffers over, ``kv_fp8_fused/fused.py:56-63``); the paged caches have their own kernels
(:mod:`economize_amd.paged`, :mod:`economize_amd.kivi`). Every call runs on the GPU; there is no CPU path.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .errors import ConfigError
from .paged import cached_workspace

__all__ = ["FP8_DTYPES", "decode_attention", "mask_operand", "sinks_operand"]

#: Query dtypes the kernels compute in.
DOT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)

def dense_counter_bytes(batch: int, queries: int, q_heads: int, kv_heads: int) -> int:
    """Bytes of the counters at the start of a dense decode workspace: int32 per batch row, KV head and block of 16
    query rows, padded to 256 bytes. They must be zero when a call starts; a call leaves them zero."""
    blocks = batch * kv_heads * -(-(q_heads // kv_heads) * queries // 16)
    return (4 * blocks + 255) // 256 * 256


def _workspace(nbytes: int, device: torch.device, batch: int, queries: int, q_heads: int,
               kv_heads: int) -> torch.Tensor:
    """The workspace of ``device``'s current stream for a dense decode call of this shape, its counters zero."""
    return cached_workspace(nbytes, dense_counter_bytes(batch, queries, q_heads, kv_heads), device)


def mask_operand(mask: torch.Tensor | None, keys: int) -> tuple[torch.Tensor | None, tuple[int, int, int, int]]:
    """The mask as the kernel reads it (one byte per element) and its ``(batch, head, query, key)`` strides with 0 on
    broadcast axes (attention/decode.py:333-349)."""
    if mask is None:
        return None, (0, 0, 0, 0)
    if mask.dtype != torch.bool:
        raise ConfigError("decode_attention takes a boolean mask")
    if mask.dim() != 4:
        raise ConfigError(f"the mask must be [B, 1 or Hq, Q or 1, S], got {tuple(mask.shape)}")
    m = mask.view(torch.uint8)
    strides = [m.stride(0), m.stride(1), m.stride(2), m.stride(3)]
    for axis in range(3):
        if m.shape[axis] == 1:
            strides[axis] = 0
    if m.shape[3] != keys:
        raise ConfigError(f"mask covers {m.shape[3]} keys, the buffer {keys}")
    return m, tuple(strides)


def sinks_operand(sinks: torch.Tensor | None, q_heads: int) -> torch.Tensor | None:
    """Attention-sink logits as one contiguous fp32 ``[Hq]`` vector (checked), or ``None`` (decode.py:352-358)."""
    if sinks is None:
        return None
    if sinks.numel() != q_heads:
        raise ConfigError(f"{sinks.numel()} sink logits for {q_heads} query heads")
    return sinks.reshape(-1).float().contiguous()


def _channel_contiguous(x: torch.Tensor) -> torch.Tensor:
    """``x`` with a contiguous last axis, 16-byte aligned rows and base (a copy only when it has not)."""
    es = x.element_size()
    if x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in x.stride()[:-1]):
        return x
    return x.contiguous()


def decode_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
                     scale: float, softcap: float | None = None, out: torch.Tensor | None = None,
                     sinks: torch.Tensor | None = None, launch: object = None, window: int | None = None,
                     k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Attention of a few queries per row over a KV buffer (attention/decode.py:252-324).

    Args:
        query: ``[B, Hq, Q, D]`` (any strides), bf16, fp16 or fp32.
        key: ``[B, Hkv, S, D]`` (any strides), the query's dtype or an fp8 dtype.
        value: ``[B, Hkv, S, Dv]``, like ``key``.
        mask: Boolean ``[B, 1 or Hq, Q or 1, S]`` (broadcast strides allowed, ``True`` = visible) or ``None``.
        scale: Multiplier of the scores.
        softcap: Optional tanh soft cap of the scaled scores.
        out: Optional ``[B, Q, Hq, Dv]`` output buffer in the query's dtype.
        sinks: Optional ``[Hq]`` attention-sink logits.
        launch: The reference's launch-plan override; the plan here is a function of the shapes, so it is ignored.
        window: The layer's sliding window, if the mask restricts every query to it (the mask alone decides what
            each query sees).
        k_scale, v_scale: Optional fp32 ``[Hkv]`` scales of fp8 K/V (this path's per-head scale mode).

    Returns:
        ``[B, Q, Hq, Dv]`` in the query's dtype (zeros for a query that sees no key).
    """
    del launch, window
    device = _lib.require_gpu(query, key, value)
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ConfigError("decode_attention takes [B, Hq, Q, D] queries and [B, Hkv, S, D] keys and values")
    batch, q_heads, queries, head_dim = query.shape
    _, kv_heads, keys, _ = key.shape
    head_dv = value.shape[-1]
    if key.shape[:3] != value.shape[:3] or key.shape[0] != batch or key.shape[3] != head_dim:
        raise ConfigError(f"K {tuple(key.shape)} / V {tuple(value.shape)} do not match the query {tuple(query.shape)}")
    if q_heads % kv_heads:
        raise ConfigError(f"{q_heads} query heads are not a multiple of {kv_heads} KV heads")
    if query.dtype not in DOT_DTYPES:
        raise ConfigError(f"decode_attention does not support {query.dtype} queries")
    if key.dtype in FP8_DTYPES:
        if value.dtype != key.dtype:
            raise ConfigError(f"K/V dtypes {key.dtype} / {value.dtype} differ")
    elif key.dtype != query.dtype or value.dtype != key.dtype:
        raise ConfigError(f"K/V dtype {key.dtype} / {value.dtype} does not match the query's {query.dtype}")
    if (k_scale is not None or v_scale is not None) and key.dtype not in FP8_DTYPES:
        raise ConfigError("per-head scales apply to fp8 K/V")
    m, mask_strides = mask_operand(mask, keys)
    sinks = sinks_operand(sinks, q_heads)
    if out is not None and (out.shape != (batch, queries, q_heads, head_dv) or out.dtype != query.dtype or
                            out.stride(-1) != 1):
        raise ConfigError("out must be [B, Q, Hq, Dv] in the query's dtype with a contiguous last axis")
    if keys == 0:  # no key: every query gives 0 (decode.py:17)
        return torch.zeros(batch, queries, q_heads, head_dv, dtype=query.dtype, device=device) if out is None \
            else out.zero_()
    query, key, value = _channel_contiguous(query), _channel_contiguous(key), _channel_contiguous(value)
    if out is None:
        out = torch.empty(batch, queries, q_heads, head_dv, dtype=query.dtype, device=device)
    need = int(_lib.lib().eco_decode_workspace_size(batch, queries, q_heads, kv_heads, keys, head_dim, head_dv))
    if need == 0:
        raise ConfigError(f"decode_attention supports head dims up to 512, got {head_dim} / {head_dv}")
    ws = _workspace(need, device, batch, queries, q_heads, kv_heads)
    ks = None if k_scale is None else k_scale.float().contiguous()
    vs = None if v_scale is None else v_scale.float().contiguous()
    _lib.call(
        "eco_decode", query.data_ptr(), _lib.fmt(query.dtype), query.stride(0), query.stride(1), query.stride(2),
        key.data_ptr(), value.data_ptr(), _lib.fmt(key.dtype), key.stride(0), key.stride(1), key.stride(2),
        value.stride(0), value.stride(1), value.stride(2), _lib.ptr(ks), _lib.ptr(vs), _lib.ptr(m), *mask_strides,
        _lib.ptr(sinks), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), batch, queries, q_heads,
        kv_heads, keys, head_dim, head_dv, float(scale if scale is not None else 1 / math.sqrt(head_dim)),
        float(softcap or 0.0), ws.data_ptr(), ws.numel(), _lib.stream_of(device),
    )
    return out
