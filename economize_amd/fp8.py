"""fp8 K/V in dense buffers on the GPU: encode with the reference's scale modes and calibrate static scales.

The reference's ``FP8Cache`` (techniques/kv_quant/fp8.py:143-217) keeps a layer's K/V as fp8 codes in dense
``[B, Hkv, S, D]`` buffers, encoded by ``fp8_encode`` (fp8.py:81-86) with no scale, a per-token scale (``token_scale``,
fp8.py:95-97) or a static per-layer scale calibrated on data (``calibrate_kv_absmax`` + ``static_scales``,
fp8.py:100-133); the fused variant hands the fp8 buffers to the attention kernel (kv_fp8_fused/fused.py:56-63). Here the
encode is the ``eco_fp8_encode`` kernel and the absolute maxima come from ``eco_kv_head_absmax``; the paged fp8 cache
(:mod:`economize_amd.paged`) serves the models its kernels take.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from . import _lib
from .errors import ConfigError

__all__ = ["FP8_MAX", "calibrate_kv_absmax", "fp8_encode", "head_absmax", "static_scales"]

#: Largest finite value of each fp8 format.
FP8_MAX = {torch.float8_e4m3fn: 448.0, torch.float8_e5m2: 57344.0}


def fp8_encode(x: torch.Tensor, dtype: torch.dtype, out: torch.Tensor | None = None,
               head_scale: torch.Tensor | None = None, token_scale: torch.Tensor | None = None) -> torch.Tensor:
    """fp8 codes of ``x`` ``[B, H, T, D]`` (bf16, fp16 or fp32, contiguous channels), as the reference's
    ``fp8_encode``: ``x / scale`` with IEEE division, clamped to the format's maximum, rounded to nearest even.

    Args:
        x: The K or V states.
        dtype: ``torch.float8_e4m3fn`` or ``torch.float8_e5m2``.
        out: Optional ``[B, H, T, D]`` fp8 destination (a view into a cache buffer, contiguous channels).
        head_scale: Optional fp32 ``[H]``: one scale per head (the static ``"tensor"`` scale repeated, or per-head
            scales).
        token_scale: Optional fp32 ``[B, H, T]`` output selecting the per-token mode: it receives each row's
            ``max(absmax / format max, 1e-12)`` (``token_scale``) and the row is encoded with it.

    Returns:
        ``out`` (or a new tensor) holding the codes.
    """
    device = _lib.require_gpu(x)
    if dtype not in FP8_MAX:
        raise ConfigError(f"fp8_encode writes float8_e4m3fn or float8_e5m2, not {dtype}")
    if x.dim() != 4 or x.dtype not in (torch.bfloat16, torch.float16, torch.float32) or x.stride(3) != 1:
        raise ConfigError("fp8_encode takes bf16 / fp16 / fp32 [B, H, T, D] states with contiguous channels")
    batch, heads, tokens, dim = x.shape
    if out is None:
        out = torch.empty(x.shape, dtype=dtype, device=device)
    if out.shape != x.shape or out.dtype != dtype or out.stride(3) != 1:
        raise ConfigError(f"out must be {dtype} {tuple(x.shape)} with contiguous channels")
    if head_scale is not None:
        head_scale = head_scale.reshape(-1).float().contiguous()
        if head_scale.numel() != heads:
            raise ConfigError(f"{head_scale.numel()} head scales for {heads} heads")
    strides = (0, 0, 0)
    if token_scale is not None:
        if token_scale.shape != (batch, heads, tokens) or token_scale.dtype != torch.float32:
            raise ConfigError(f"token_scale must be fp32 {(batch, heads, tokens)}")
        strides = token_scale.stride()
    _lib.call("eco_fp8_encode", x.data_ptr(), _lib.fmt(x.dtype), x.stride(0), x.stride(1), x.stride(2),
              out.data_ptr(), _lib.fmt(dtype), out.stride(0), out.stride(1), out.stride(2), batch, heads, tokens,
              dim, _lib.ptr(head_scale), _lib.ptr(token_scale), *strides, _lib.stream_of(device))
    return out


def head_absmax(x: torch.Tensor, into: torch.Tensor) -> torch.Tensor:
    """Max-accumulate each head's absolute maximum of ``x`` ``[B, H, S, D]`` into ``into`` (int32 ``[H]`` holding
    float bit patterns, zero at the start), on the GPU."""
    device = _lib.require_gpu(x, into)
    b, h, s, d = x.shape
    if into.shape != (h,) or into.dtype != torch.int32:
        raise ConfigError(f"head_absmax accumulates into int32 [{h}]")
    _lib.call("eco_kv_head_absmax", x.data_ptr(), _lib.fmt(x.dtype), b, h, s, d, *x.stride(), into.data_ptr(),
              _lib.stream_of(device))
    return into


def static_scales(absmax: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``absmax / format max``, 1 where that is not positive (fp8.py:130-133); fp32, same shape."""
    scales = absmax.float() / FP8_MAX[dtype]
    return torch.where(scales > 0, scales, torch.ones_like(scales))


@torch.no_grad()
def calibrate_kv_absmax(model: torch.nn.Module, batches: Sequence[torch.Tensor], per_head: bool = False
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    """The absolute maxima of the keys and values every layer writes into its cache on ``batches`` (the reference's
    ``calibrate_kv_absmax``, fp8.py:100-127): the model runs each batch with a cache that records the states it
    receives. Returns fp32 ``(keys, values)`` on the CPU, ``[layers]``, or ``[layers, Hkv]`` with ``per_head``;
    a layer that never writes its cache keeps 0."""
    from transformers import DynamicCache

    layers = model.config.num_hidden_layers
    kv_heads = getattr(model.config, "num_key_value_heads", None) or model.config.num_attention_heads
    device = next(model.parameters()).device
    bits = torch.zeros(2, layers, kv_heads, dtype=torch.int32, device=device)

    class Recording(DynamicCache):
        def update(self, key_states, value_states, layer_idx, *args, **kwargs):
            head_absmax(key_states, bits[0, layer_idx])
            head_absmax(value_states, bits[1, layer_idx])
            return super().update(key_states, value_states, layer_idx, *args, **kwargs)

    for batch in batches:
        model(input_ids=batch.to(device), past_key_values=Recording(config=model.config), use_cache=True)
    absmax = bits.view(torch.float32).cpu()
    if not per_head:
        absmax = absmax.amax(dim=2)
    return absmax[0], absmax[1]
