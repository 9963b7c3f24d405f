"""The ``"economize"`` attention kernel registration and its forward over the paged caches.

Follows attention/registry.py:36-81 (``AttentionKernel``, ``ATTENTION_KERNELS``, ``accepts_fp8_kv``,
``accepts_packed_kv``) and attention/interface.py:416-499 (``economize_attention_forward`` and the
``ATTENTION_KERNELS.register("economize", ...)`` call).

The reference's forward receives dense K/V tensors and reads a packed format from an object attached to the key
(attention/packed.py:61-63). Here the layer's K/V live in a paged cache only, so the ``key`` argument is a
:class:`PagedKV` handle: the cache, its block table, the row lengths and, for Quest, the page bounds. The forward
dispatches on its format:

* ``"fp8"`` / ``"bf16"``: :class:`~economize_amd.paged.PagedKVCache` ->
  :func:`~economize_amd.paged.paged_decode_attention`;
* ``"quest"``: a :class:`~economize_amd.paged.PagedKVCache` with :class:`~economize_amd.quest.QuestPages` ->
  :meth:`~economize_amd.quest.QuestPages.attend` (dense past ``max_queries``, as attention/quest.py:191-204);
* ``"kivi"``: :class:`~economize_amd.kivi.PagedKIVICache` -> :func:`~economize_amd.kivi.kivi_decode_attention`.

Like the reference's forward it takes the query ``[B, Hq, Q, D]``, the soft cap from ``kwargs["softcap"]`` and the
sinks from ``kwargs["s_aux"]`` or ``kwargs["sinks"]`` (attention/interface.py:179-184), and returns
``(out [B, Q, Hq, D], None)``.
"""

from __future__ import annotations

from collections import Counter
from collections.abc import Callable
from dataclasses import dataclass

import torch

from .errors import ConfigError
from .kivi import PagedKIVICache, kivi_decode_attention
from .paged import PagedKVCache, paged_decode_attention
from .quest import QuestPages
from .techniques import Registry

__all__ = ["ATTENTION_KERNELS", "AttentionKernel", "PACKED_FORMATS", "PagedKV", "accepts_fp8_kv",
           "accepts_packed_kv", "economize_attention_forward", "kernel_calls"]

#: Packed formats the ``"economize"`` kernel reads (the reference's set less ``"gathered"``, a dense gather that the
#: paged page list replaces).
PACKED_FORMATS = frozenset({"kivi", "quest"})


@dataclass(frozen=True)
class AttentionKernel:
    """A registered attention implementation (attention/registry.py:36-67)."""

    family: str
    forward: Callable[..., tuple[torch.Tensor, torch.Tensor | None]]
    mask_function: Callable[..., object] | None = None
    description: str = ""
    fp8_kv: bool = False
    packed_kv: frozenset[str] = frozenset()
    sparse_prefill: bool = False
    structured_masks: bool = False


ATTENTION_KERNELS: Registry = Registry("attention kernel")


def accepts_fp8_kv(implementation: str) -> bool:
    """Whether the registered kernel ``implementation`` takes fp8 K/V directly."""
    return implementation in ATTENTION_KERNELS and ATTENTION_KERNELS[implementation].fp8_kv


def accepts_packed_kv(implementation: str, fmt: str) -> bool:
    """Whether the registered kernel ``implementation`` reads packed K/V of format ``fmt``."""
    return implementation in ATTENTION_KERNELS and fmt in ATTENTION_KERNELS[implementation].packed_kv


@dataclass(frozen=True)
class PagedKV:
    """One layer's paged K/V as the forward reads it.

    Attributes:
        cache: A :class:`~economize_amd.paged.PagedKVCache` or :class:`~economize_amd.kivi.PagedKIVICache`.
        block_table: int32 ``[B, pages per row]``.
        seq_lens: int32 ``[B]`` tokens of every row, the queries' own included.
        max_seq_len: Bound of ``seq_lens`` on the host.
        pages: Quest page bounds of a :class:`~economize_amd.paged.PagedKVCache`, or ``None``.
    """

    cache: PagedKVCache | PagedKIVICache
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    max_seq_len: int
    pages: QuestPages | None = None

    def __post_init__(self) -> None:
        if self.pages is not None and not isinstance(self.cache, PagedKVCache):
            raise ConfigError("Quest pages index a paged fp8 or bf16 cache")
        if not isinstance(self.cache, (PagedKVCache, PagedKIVICache)):
            raise ConfigError(f"no economize kernel reads a {type(self.cache).__name__}")

    @property
    def format(self) -> str:
        if isinstance(self.cache, PagedKIVICache):
            return "kivi"
        if self.pages is not None:
            return "quest"
        return "bf16" if self.cache.dtype == torch.bfloat16 else "fp8"


_calls: Counter = Counter()


def kernel_calls() -> dict[str, int]:
    """Calls of :func:`economize_attention_forward` by format since the process started."""
    return dict(_calls)


def economize_attention_forward(module: torch.nn.Module | None, query: torch.Tensor, key: PagedKV,
                                value: object = None, attention_mask: torch.Tensor | None = None,
                                dropout: float = 0.0, scaling: float | None = None, is_causal: bool | None = None,
                                **kwargs: object) -> tuple[torch.Tensor, None]:
    """Decode attention of ``query`` ``[B, Hq, Q, D]`` (bf16) over the paged K/V that ``key`` describes; returns
    ``(out [B, Q, Hq, D] bf16, None)``. The ``Q`` queries are the last ``Q`` tokens of every row and see keys
    causally. ``value`` is unused (the cache holds both); a mask tensor and dropout are refused, since the paged
    kernels take visibility from the row lengths."""
    if not isinstance(key, PagedKV):
        raise ConfigError("the economize kernel reads a PagedKV handle, not dense K/V tensors")
    if attention_mask is not None:
        raise ConfigError("the paged kernels take causal visibility from seq_lens, not an attention mask")
    if dropout:
        raise ConfigError("decode attention has no dropout")
    if query.dim() != 4:
        raise ConfigError(f"query must be [B, Hq, Q, D], got {tuple(query.shape)}")
    softcap = kwargs.get("softcap")
    sinks = kwargs.get("s_aux") if kwargs.get("s_aux") is not None else kwargs.get("sinks")
    fmt = key.format
    if fmt == "kivi":
        out = kivi_decode_attention(query.transpose(1, 2), key.cache, key.block_table, key.seq_lens, key.max_seq_len,
                                    scaling, softcap, sinks)
    elif fmt == "quest":
        out = key.pages.attend(query, key.cache, key.block_table, key.seq_lens, key.max_seq_len, scaling, softcap,
                               sinks)
    else:
        out = paged_decode_attention(query.transpose(1, 2), key.cache, key.block_table, key.seq_lens,
                                     key.max_seq_len, scaling, softcap, sinks)
    _calls[fmt] += 1
    return out, None


ATTENTION_KERNELS.register("economize", AttentionKernel(
    family="sdpa", forward=economize_attention_forward,
    description="MI355X decode attention over paged fp8 / bf16 / KIVI caches, with Quest page selection",
    fp8_kv=True, packed_kv=PACKED_FORMATS,
))
