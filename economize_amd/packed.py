"""Packed K/V handed to the attention function on the key tensor (the reference's attention/packed.py:25-78).

A cache that stores a layer in a format an attention kernel reads directly (here: the paged fp8 / bf16 cache, the
paged KIVI cache, Quest's pages over a paged cache) returns stand-ins for the layer's dense K/V and attaches the
format's handle to a fresh view of the key; a cache that keeps dense buffers but lets the kernel read less of them
(Quest's pages over a dense cache, an eviction's kept entries) attaches its handle to the key buffer's view itself.
:func:`economize_amd.attention.economize_attention_forward` finds the handle with :func:`packed_of` and calls its
``attend``; an attention function that does not read the format calls :func:`materialized_kv`, which builds the
dense K/V through the handle's ``materialize`` (the gather kernels), and applies the handle's ``restrict_mask`` when
it has one, so the fallbacks compute the same attention. The handle is an attribute of one view object only: any new
tensor made from the key (a copy, a slice, a reordering of rows) is a different object without it, so a handle can
only ever be read together with the exact tensor it was attached to.
"""

from __future__ import annotations

from typing import Protocol, runtime_checkable

import torch

__all__ = ["PackedKV", "attach_packed", "materialized_kv", "packed_of", "stand_in"]

_ATTR = "_economize_packed"


@runtime_checkable
class PackedKV(Protocol):
    """Packed K/V of one layer that a kernel attends over directly (attention/packed.py:29-51)."""

    #: Format name, matched against :attr:`~economize_amd.attention.AttentionKernel.packed_kv`.
    format: str

    def attend(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, mask: torch.Tensor | None,
               scale: float, softcap: float | None = None, sinks: torch.Tensor | None = None) -> torch.Tensor:
        """Attention of ``query`` ``[B, Hq, Q, D]`` over the layer's cache, ``[B, Q, Hq, Dv]`` out."""
        ...


def attach_packed(key: torch.Tensor, packed: object) -> torch.Tensor:
    """``key`` as a new view object with ``packed`` as its attribute; ``key`` and its storage are not modified."""
    view = key.view(key.shape)
    setattr(view, _ATTR, packed)
    return view


def packed_of(key: object) -> object | None:
    """The handle attached to ``key``, or ``None``."""
    return getattr(key, _ATTR, None)


def materialized_kv(key: torch.Tensor, value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``key`` and ``value`` as dense tensors an attention function without the packed kernel can read: the
    attachment's ``materialize()`` when it has one, else ``key`` and ``value`` unchanged. The materialized key keeps
    the attachment (attention/packed.py:66-78)."""
    packed = packed_of(key)
    build = getattr(packed, "materialize", None)
    if packed is None or build is None:
        return key, value
    dense_key, dense_value = build()
    return attach_packed(dense_key, packed), dense_value


def stand_in(shape: tuple[int, ...], dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A zero-memory tensor of ``shape``: one element broadcast over every index (the place of a layer's dense K/V
    that the cache does not keep)."""
    return torch.zeros((), dtype=dtype, device=device).expand(*shape)
