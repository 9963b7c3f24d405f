"""The ``"economize"`` attention kernel: its registration, the transformers attention function and ``install``.

Follows attention/registry.py:36-81 (``AttentionKernel``, ``ATTENTION_KERNELS``, ``accepts_fp8_kv``,
``accepts_packed_kv``) and attention/interface.py:243-525 (``economize_attention_forward`` with its per-call fallback
reasons, ``kernel_calls`` / ``kernel_usage`` / ``usage_summary``, the registration and ``install``).

:func:`economize_attention_forward` takes transformers' arguments: ``query`` ``[B, Hq, Q, D]``, ``key`` / ``value``
``[B, Hkv, S, D]`` and an optional boolean mask ``[B, 1 or Hq, Q, >= S]``, and returns ``([B, Q, Hq, Dv], None)``.

* A key that carries a paged cache's handle (:class:`PagedKV`, attached by :mod:`economize_amd.hf`'s cache; see
  :mod:`economize_amd.packed`) attends over the paged fp8 / bf16 cache, its Quest pages or the paged KIVI cache on the
  paged kernels (path ``"kernel_<format>"``).
* Dense K/V (bf16 / fp16 / fp32, or fp8 views of an fp8 cache) attend on the dense decode kernel
  (:func:`economize_amd.decode.decode_attention`, path ``"kernel"``); with a :class:`~economize_amd.gathered.GatheredKV`
  attached (an eviction's compacted prompt entries), over the compact entries and the dense tail (path
  ``"kernel_gathered"``); with :class:`~economize_amd.quest.QuestPages` attached, over the selected pages and the
  dense tail (path ``"kernel_quest"``).
* Everything else falls back per call to transformers' ``sdpa`` (a paged cache's K/V materialized by the gather
  kernels first, fp8 K/V upcast to the query's dtype, Quest's unselected pages hidden in the mask as the reference's
  fallback hides them, interface.py:216-222), or to the model's eager function when the call has sinks or asks for
  the weights: long queries (prefill), CPU tensors, training with dropout, ``output_attentions``, other dtypes, masks
  that are not boolean ``[B, 1 or Hq, Q, S]``.
"""

from __future__ import annotations

import sys
from collections import Counter
from collections.abc import Callable
from dataclasses import dataclass
from typing import TypedDict

import torch

from .decode import FP8_DTYPES, decode_attention
from .errors import ConfigError
from .kivi import PagedKIVICache, kivi_decode_attention, kivi_gather
from .packed import materialized_kv, packed_of
from .paged import PagedKVCache, paged_decode_attention, paged_gather
from .quest import QuestPages
from .techniques import Registry

__all__ = ["ATTENTION_KERNELS", "MAX_QUERIES", "NAME", "PACKED_FORMATS", "AttentionKernel", "PagedKV",
           "accepts_fp8_kv", "accepts_packed_kv", "economize_attention_forward", "install", "kernel_calls",
           "kernel_usage", "usage_summary"]

#: Name of the implementation in transformers and in :data:`ATTENTION_KERNELS`.
NAME = "economize"
#: Longest query (tokens per row) the kernels take; longer ones (prefill) fall back to ``sdpa``.
MAX_QUERIES = 64
#: Packed formats the ``"economize"`` kernel reads (the reference's set, interface.py:70, plus the paged fp8 / bf16
#: cache).
PACKED_FORMATS = frozenset({"kivi", "gathered", "quest", "fp8", "bf16"})

_DOT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


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
    """One layer's paged K/V, attached to the key the cache returns (or passed as the key itself).

    Attributes:
        cache: A :class:`~economize_amd.paged.PagedKVCache` or :class:`~economize_amd.kivi.PagedKIVICache`.
        block_table: int32 ``[B, pages per row]``.
        seq_lens: int32 ``[B]`` tokens of every row, the queries' own included.
        max_seq_len: Bound of ``seq_lens`` on the host.
        pages: Quest page bounds of a :class:`~economize_amd.paged.PagedKVCache`, or ``None``.
        dtype: The model's dtype (of the dense view :meth:`materialize` builds).
        current: For :meth:`materialize`: the dense K/V ``[B, Hkv, T, D]`` of the pass that is writing the last ``T``
            tokens, when they are to be read as the pass computed them (KIVI quantizes a pass's tokens only at its
            end), else ``None``.
        static: ``max_seq_len`` is the cache's capacity, not the rows' length (a static cache's reads have fixed
            shapes): the dense view is capacity-long, and a fallback without a mask hides the slots past each
            row's ``seq_lens`` (:meth:`visible_mask`).
    """

    cache: PagedKVCache | PagedKIVICache
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    max_seq_len: int
    pages: QuestPages | None = None
    dtype: torch.dtype = torch.bfloat16
    current: tuple[torch.Tensor, torch.Tensor] | None = None
    static: bool = False

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

    def attend(self, query: torch.Tensor, key: torch.Tensor | None, value: torch.Tensor | None,
               mask: torch.Tensor | None, scale: float | None, softcap: float | None = None,
               sinks: torch.Tensor | None = None) -> torch.Tensor:
        """``[B, Q, Hq, D]`` attention of ``query`` ``[B, Hq, Q, D]`` over the paged cache: the ``Q`` queries
        are the last ``Q`` tokens of every row (causal), and ``mask`` (boolean ``[B or 1, Hq or 1, Q or 1, >= S]``,
        key ``t`` = token ``t``) hides keys on top."""
        q = query.transpose(1, 2)
        if self.format == "kivi":
            return kivi_decode_attention(q, self.cache, self.block_table, self.seq_lens, self.max_seq_len, scale,
                                         softcap, sinks, mask=mask)
        if self.format == "quest":
            return self.pages.attend_paged(query, self.cache, self.block_table, self.seq_lens, self.max_seq_len,
                                           scale, softcap, sinks, mask=mask)
        return paged_decode_attention(q, self.cache, self.block_table, self.seq_lens, self.max_seq_len, scale,
                                      softcap, sinks, mask=mask)

    def restrict_mask(self, query: torch.Tensor, key: torch.Tensor, mask: torch.Tensor | None,
                      is_causal: bool = False) -> torch.Tensor | None:
        """For a fallback over the materialized K/V: ``mask`` with the pages Quest does not select hidden
        (:meth:`~economize_amd.quest.QuestPages.restrict_mask`), or ``mask`` itself without Quest pages."""
        if self.pages is None:
            return mask
        return self.pages.restrict_mask(query, key, mask, is_causal)

    def visible_mask(self, queries: int) -> torch.Tensor:
        """Boolean ``[B, 1, Q, max_seq_len]``: key ``t`` visible to query ``qi`` of row ``b`` when
        ``t < seq_lens[b] - Q + qi + 1`` (the causal rule of the paged kernels), from the device lengths."""
        t = torch.arange(self.max_seq_len, device=self.seq_lens.device).view(1, 1, 1, -1)
        qi = torch.arange(queries, device=self.seq_lens.device).view(1, 1, -1, 1)
        return t < self.seq_lens.view(-1, 1, 1, 1) - queries + qi + 1

    def materialize(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The dense K/V ``[B, Hkv, max_seq_len, D]`` the kernels read, in :attr:`dtype` (the gather kernels)."""
        past = self.max_seq_len - (self.current[0].shape[2] if self.current is not None else 0)
        gather = kivi_gather if isinstance(self.cache, PagedKIVICache) else paged_gather
        k, v = gather(self.cache, self.block_table, past if self.current is not None else self.max_seq_len,
                      self.dtype)
        if self.current is not None:
            k = torch.cat([k, self.current[0].to(self.dtype)], dim=2)
            v = torch.cat([v, self.current[1].to(self.dtype)], dim=2)
        return k, v


# ---- usage log (attention/interface.py:89-137) -------------------------------------------------------------------


class UsageRecord(TypedDict):
    layer: int | None
    queries: int
    path: str
    reason: str
    calls: int


_calls = {"kernel": 0, "fallback": 0}
_usage: Counter = Counter()


def kernel_calls() -> dict[str, int]:
    """How many attention calls ran on the kernels and on the fallback since import."""
    return dict(_calls)


def kernel_usage(reset: bool = False) -> list[UsageRecord]:
    """Which path each attention call took, grouped by layer, query length and fallback reason."""
    rows: list[UsageRecord] = [{"layer": layer, "queries": queries, "path": path, "reason": reason, "calls": n}
                               for (layer, queries, path, reason), n in _usage.items()]
    rows.sort(key=lambda r: (-1 if r["layer"] is None else r["layer"], r["queries"], r["path"], r["reason"]))
    if reset:
        _usage.clear()
    return rows


def usage_summary() -> dict:
    """Calls per path, per fallback reason, and the query lengths per path."""
    paths: Counter = Counter()
    reasons: Counter = Counter()
    lengths: dict[str, set[int]] = {}
    for (_, queries, path, reason), n in _usage.items():
        paths[path] += n
        if not path.startswith("kernel"):
            reasons[reason] += n
        lengths.setdefault(path, set()).add(queries)
    return {"calls": dict(paths), "fallback_reasons": dict(reasons),
            "queries": {path: sorted(q) for path, q in lengths.items()}}


# ---- the forward ---------------------------------------------------------------------------------------------------


def _sinks(kwargs: dict) -> object:
    return kwargs.get("s_aux") if kwargs.get("s_aux") is not None else kwargs.get("sinks")


def _fallback_reason(module, query: torch.Tensor, key, attention_mask, dropout: float, kwargs: dict,
                     paged: PagedKV | None, gathered: object = None) -> str | None:
    """Why this call cannot run on the kernels, or ``None`` when it can; decided per call (interface.py:243-285)."""
    batch, q_heads, queries, _ = query.shape
    if not query.is_cuda:
        return "cpu"
    if queries > MAX_QUERIES:
        return "long_query"
    if dropout > 0.0 and module is not None and module.training:
        return "dropout"
    sinks = _sinks(kwargs)
    if sinks is not None and (not torch.is_tensor(sinks) or sinks.numel() != q_heads):
        return "sinks"
    if kwargs.get("output_attentions", False):
        return "output_attentions"
    if query.dtype not in _DOT_DTYPES:
        return "dtype"
    if paged is not None:
        if query.dtype != torch.bfloat16 and not (query.dtype == torch.float16 and paged.format == "fp8"):
            return "dtype"  # the paged kernels take bf16 queries, and fp16 ones over an fp8 cache
        kv_heads = paged.cache.kv_heads
        if q_heads % kv_heads == 0 and q_heads // kv_heads > 64:
            return "heads_per_kv"  # the paged kernels take at most 64 query heads per KV head
    else:
        if key.dtype != query.dtype and (key.dtype not in FP8_DTYPES or gathered is not None):
            return "kv_dtype"  # the gathered kernel takes K/V in the query's dtype
        kv_heads = key.shape[1]
    if q_heads % kv_heads:
        return "heads"
    if attention_mask is None:
        return None if queries == 1 or paged is not None else "no_mask"  # the paged kernels are causal by length
    if not torch.is_tensor(attention_mask) or attention_mask.dtype != torch.bool:
        return "float_mask"
    if attention_mask.dim() != 4:
        return "mask_rank"
    m_batch, m_heads, m_queries, m_keys = attention_mask.shape
    if m_batch not in (1, batch) or m_heads not in (1, q_heads) or m_queries not in (1, queries):
        return "mask_shape"
    keys = paged.max_seq_len if paged is not None else key.shape[2]
    if m_keys < keys:
        return "mask_keys"
    return None


def _eager_function(module, kwargs: dict):
    """The model's own ``eager_attention_forward`` when the call needs it (sinks, attention weights), which ``sdpa``
    does not compute (interface.py:194-203)."""
    if _sinks(kwargs) is None and not kwargs.get("output_attentions", False):
        return None
    return getattr(sys.modules.get(type(module).__module__), "eager_attention_forward", None)


def _fallback(module, query, key, value, attention_mask, dropout, scaling, is_causal, reason, kwargs):
    """One call on transformers' ``sdpa`` (or the model's eager function for sinks and weights), over the dense K/V:
    a paged cache's gathered by its handle, fp8 ones upcast to the query's dtype (interface.py:206-240)."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    layer = getattr(module, "layer_idx", None)
    handle = packed_of(key)
    key, value = materialized_kv(key, value)
    if torch.is_tensor(attention_mask) and attention_mask.dim() == 4 and attention_mask.shape[-1] > key.shape[2]:
        attention_mask = attention_mask[..., : key.shape[2]]
    if attention_mask is None and getattr(handle, "static", False):  # capacity-long K/V: hide the unwritten slots
        attention_mask, is_causal = handle.visible_mask(query.shape[2]), False
    restrict = getattr(packed_of(key), "restrict_mask", None)
    if restrict is not None:  # a sparse cache (Quest) hides what its kernel would not read (interface.py:216-222)
        restricted = restrict(query, key, attention_mask, bool(is_causal))
        if restricted is not attention_mask:
            attention_mask, is_causal = restricted, False
    if key.dtype in FP8_DTYPES:
        key, value = key.to(query.dtype), value.to(query.dtype)
    _calls["fallback"] += 1
    eager = _eager_function(module, kwargs)
    if eager is None:
        _usage[(layer, query.shape[2], "sdpa", reason)] += 1
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      is_causal=is_causal, **kwargs)
    _usage[(layer, query.shape[2], "eager", reason)] += 1
    mask = attention_mask
    if mask is not None and mask.dtype == torch.bool:  # eager functions add the mask to the scores
        mask = torch.zeros(mask.shape, dtype=query.dtype, device=query.device).masked_fill(
            ~mask, torch.finfo(query.dtype).min)
    scale = query.shape[-1] ** -0.5 if scaling is None else scaling
    return eager(module, query, key, value, mask, scaling=scale, dropout=dropout, **kwargs)


def economize_attention_forward(module: torch.nn.Module | None, query: torch.Tensor, key, value,
                                attention_mask: torch.Tensor | None, dropout: float = 0.0,
                                scaling: float | None = None, is_causal: bool | None = None,
                                **kwargs: object) -> tuple[torch.Tensor, torch.Tensor | None]:
    """transformers attention function (``[B, Hq, Q, D]`` in, ``[B, Q, Hq, Dv]`` out) on the MI355X kernels
    (interface.py:416-480); the kernel or the fallback is chosen for every call, and :func:`kernel_usage` logs it.
    ``key`` may also be a :class:`PagedKV` itself (then ``value`` is unused)."""
    if query.dim() != 4:
        raise ConfigError(f"query must be [B, Hq, Q, D], got {tuple(query.shape)}")
    handle = key if isinstance(key, PagedKV) else packed_of(key)
    paged = handle if isinstance(handle, PagedKV) else None
    # packed K/V over dense buffers: a gathered cache's compact entries, Quest's pages of a dense cache, KIVI codes in
    # the reference's layout
    dense_packed = handle if paged is None and getattr(handle, "format", None) in ("gathered", "quest", "kivi") \
        else None
    gathered = dense_packed if getattr(dense_packed, "format", None) == "gathered" else None
    layer = getattr(module, "layer_idx", None)
    queries = query.shape[2]
    reason = _fallback_reason(module, query, key, attention_mask, dropout, kwargs, paged, gathered)
    if reason is not None:
        if isinstance(key, PagedKV):
            raise ConfigError(f"a bare PagedKV handle cannot fall back ({reason}); attach it to dense stand-ins")
        return _fallback(module, query, key, value, attention_mask, dropout, scaling, is_causal, reason, kwargs)
    scale = query.shape[-1] ** -0.5 if scaling is None else scaling
    softcap = kwargs.get("softcap")
    sinks = _sinks(kwargs)
    if paged is not None:
        out = paged.attend(query, key, value, attention_mask, scale, softcap, sinks)
        path = f"kernel_{paged.format}"
    else:
        if attention_mask is not None and attention_mask.shape[-1] != key.shape[2]:
            attention_mask = attention_mask[..., : key.shape[2]]
        if dense_packed is not None:
            out = dense_packed.attend(query, key, value, attention_mask, scale, softcap, sinks)
            path = f"kernel_{dense_packed.format}"
        else:
            out = decode_attention(query, key, value, attention_mask, scale, softcap=softcap, sinks=sinks)
            path = "kernel"
    _calls["kernel"] += 1
    _usage[(layer, queries, path, "")] += 1
    return out, None


ATTENTION_KERNELS.register(NAME, AttentionKernel(
    family="sdpa", forward=economize_attention_forward,
    description="MI355X decode attention: dense bf16/fp16/fp32/fp8 K/V with masks, paged fp8/bf16 and KIVI caches, "
                "Quest pages",
    fp8_kv=True, packed_kv=PACKED_FORMATS, structured_masks=False,
))


def install(name: str | None = None) -> list[str]:
    """Register the attention kernels with transformers (``AttentionInterface`` and ``AttentionMaskInterface``,
    interface.py:502-525); afterwards ``attn_implementation="economize"`` selects the kernel. Idempotent."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    names = [name] if name is not None else ATTENTION_KERNELS.names()
    for each in names:
        entry = ATTENTION_KERNELS.get_entry(each)
        AttentionInterface.register(each, entry.forward)
        mask = entry.mask_function or AttentionMaskInterface._global_mapping[entry.family]
        AttentionMaskInterface.register(each, mask)
    return names
