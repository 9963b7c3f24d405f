"""The technique configurations of the compressed-KV path and their registry, as the reference declares them.

* :class:`FP8KVConfig` / :class:`FusedFP8KVConfig` follow techniques/kv_quant/fp8.py:55-79 and
  techniques/kv_fp8_fused/fused.py:25-49 (``"head"``, a per-KV-head absmax scale, is this path's scale mode beside the
  reference's ``"none"``, ``"token"`` and ``"tensor"``).
* :class:`KIVIConfig` / :class:`FusedKIVIConfig` follow techniques/kv_quant/kivi.py:53-107 and
  techniques/kv_kivi_fused/fused.py:30-51.
* :class:`QuestConfig` follows techniques/quest/technique.py:45-115.
* :func:`register_technique`, :data:`TECHNIQUES` and :func:`technique_for` follow core/technique.py:345-375.

A technique makes the paged layer cache its configuration describes (:meth:`Technique.make_cache`); the caches and
kernels live in :mod:`economize_amd.paged`, :mod:`economize_amd.kivi` and :mod:`economize_amd.quest`.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from numbers import Integral
from typing import ClassVar

import torch

from .errors import ConfigError, IncompatibleTechniquesError

__all__ = [
    "FP8KVConfig", "FusedFP8KVConfig", "FusedKIVIConfig", "KIVIConfig", "QuestConfig", "Registry", "TECHNIQUES",
    "Technique", "TechniqueConfig", "register_technique", "technique_for",
]

FP8_FORMATS: dict[str, torch.dtype] = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
FP8_SCALES = ("none", "token", "tensor", "head")
KIVI_BITS = (2, 4, 8)


def _choice(name: str, value, choices) -> None:
    if value not in choices:
        raise ConfigError(f"{name} must be one of {list(choices)}, got {value!r}")


def _positive(name: str, value) -> None:
    if isinstance(value, bool) or not isinstance(value, Integral) or value <= 0:
        raise ConfigError(f"{name} must be a positive integer, got {value!r}")


def _layers(layers) -> None:
    """A tuple of 1-indexed layers, empty for every layer (validation.py:64-74)."""
    if not isinstance(layers, tuple) or not all(isinstance(i, int) and not isinstance(i, bool) for i in layers):
        raise ConfigError(f"layers must be a tuple of 1-indexed layer numbers, got {layers!r}")
    if any(i < 1 for i in layers):
        raise ConfigError(f"layers are 1-indexed, got {layers!r}")


def attn_implementation(adapter) -> str:
    """The attention implementation a model runs: ``adapter`` is a model adapter, a transformers model or its config
    (whatever carries ``config._attn_implementation``, as the reference's ``validate(adapter)`` reads it), or the
    implementation's name."""
    if isinstance(adapter, str):
        return adapter
    config = getattr(adapter, "config", adapter)
    return str(getattr(config, "_attn_implementation", None) or "eager")


def head_dim_of(adapter) -> int | None:
    """The attention head dimension of a model (``head_dim``, else ``hidden_size / num_attention_heads``), or
    ``None`` when ``adapter`` names no model."""
    config = getattr(adapter, "config", adapter)
    dim = getattr(config, "head_dim", None)
    if dim is None and getattr(config, "hidden_size", None) and getattr(config, "num_attention_heads", None):
        dim = config.hidden_size // config.num_attention_heads
    return int(dim) if dim else None


def _head_dims(technique: str, adapter, dims: tuple[int, ...]) -> None:
    dim = head_dim_of(adapter)
    if dim is not None and dim not in dims:
        raise ConfigError(f"{technique}: the MI355X kernels take head dims {list(dims)}, the model has {dim}")


def _dense_head_dim(technique: str, adapter, kv_in_model_dtype: bool) -> None:
    """Refuses head dims the dense decode kernel does not take: at most 512 channels (heads wider than 256 run as two
    value slices, attention/decode.py:216-232), and at most 256 when the K/V buffers are fp32 (a model's own dtype on
    an fp32 model)."""
    dim = head_dim_of(adapter)
    if dim is None:
        return
    limit = 256 if kv_in_model_dtype and model_dtype(adapter) == torch.float32 else 512
    if dim > limit:
        raise ConfigError(f"{technique}: the MI355X kernels take head dims up to {limit} here, the model has {dim}")


def model_dtype(adapter) -> torch.dtype | None:
    """The dtype of a model's parameters, or ``None`` when ``adapter`` is no module."""
    parameters = getattr(adapter, "parameters", None)
    if parameters is None:
        return None
    first = next(iter(parameters()), None)
    return None if first is None else first.dtype


def kivi_paged_refusal(config, adapter) -> str | None:
    """Why the paged KIVI cache (32-token pages of 2- or 4-bit codes read by the fused kernel) cannot hold
    ``config``'s layers on this model, or ``None`` when it can; such layers keep the reference's packed record
    (any bits, group, head dim and dtype; :meth:`KIVIConfig.layer_kind`)."""
    if config.bits not in (2, 4):
        return f"bits={config.bits}"
    if config.group_size != 32:
        return f"group_size={config.group_size}"
    dim = head_dim_of(adapter)
    if dim is not None and dim not in (64, 128):
        return f"head dim {dim}"
    dtype = model_dtype(adapter)
    if dtype is not None and dtype != torch.bfloat16:
        return f"a {dtype} model"
    if config.headroom < 64:
        return f"headroom {config.headroom} (below 64 decoding queries)"
    return None


def _needs_kernel(technique: str, implementation: str, accepts, what: str, instead: str | None) -> None:
    """Refuses an attention implementation that cannot read the technique's cache (fused.py:44-49)."""
    from .attention import ATTENTION_KERNELS

    if not accepts(implementation):
        readers = [name for name in ATTENTION_KERNELS.names() if accepts(name)]
        tail = f" or use {instead}" if instead else ""
        raise IncompatibleTechniquesError(
            f"{technique} needs an attention kernel that reads {what}, the model runs {implementation!r}; "
            f"load it with attn_implementation in {readers}{tail}")


class Registry(dict):
    """Name -> entry, refusing a name twice (the reference's registry.Registry)."""

    def __init__(self, what: str) -> None:
        super().__init__()
        self.what = what

    def register(self, name: str, entry) -> None:
        if name in self:
            raise ConfigError(f"{self.what} {name!r} is already registered")
        self[name] = entry

    def get_entry(self, name: str):
        try:
            return self[name]
        except KeyError:
            raise ConfigError(f"unknown {self.what} {name!r}; registered: {sorted(self)}") from None

    def names(self) -> list[str]:
        return sorted(self)


# ---- configurations -----------------------------------------------------------------------------------------


class TechniqueConfig:
    """JSON round trip of a frozen configuration dataclass (core/technique.py's ``to_dict`` / ``from_dict``)."""

    technique: ClassVar[str]

    def to_dict(self) -> dict:
        out = {"technique": self.technique}
        out.update({f.name: getattr(self, f.name) for f in fields(self)})
        return out

    @classmethod
    def from_dict(cls, data: dict):
        data = dict(data)
        if data.pop("technique", cls.technique) != cls.technique:
            raise ConfigError(f"{cls.__name__} builds {cls.technique!r}, not {data.get('technique')!r}")
        known = {f.name: f for f in fields(cls)}
        unknown = sorted(set(data) - set(known))
        if unknown:
            raise ConfigError(f"unknown {cls.__name__} fields {unknown}")
        return cls(**{k: tuple(v) if isinstance(v, list) else v for k, v in data.items()})


@dataclass(frozen=True)
class FP8KVConfig(TechniqueConfig):
    """FP8 KV cache.

    Attributes:
        format: ``"e4m3"`` or ``"e5m2"``.
        scale: ``"none"``, ``"token"`` or ``"tensor"`` as in the reference, or ``"head"``: one static scale per KV
            head for the keys and one for the values (absmax over calibration data / the format's maximum).
        layers: 1-indexed layers whose cache is stored in fp8 (empty: every layer).
    """

    technique: ClassVar[str] = "kv_fp8"
    format: str = "e4m3"
    scale: str = "none"
    layers: tuple[int, ...] = ()

    def __post_init__(self) -> None:
        _choice("format", self.format, tuple(FP8_FORMATS))
        _choice("scale", self.scale, FP8_SCALES)
        _layers(self.layers)

    @property
    def dtype(self) -> torch.dtype:
        return FP8_FORMATS[self.format]

    def validate(self, adapter) -> None:
        """Every scale mode and head dim runs: the paged fp8 cache where its kernels take the model, dense fp8
        buffers decoded to the model's dtype otherwise (check_layers / check_positional of fp8.py:77-79 have no
        counterpart: layers are checked when the cache is built)."""


@dataclass(frozen=True)
class FusedFP8KVConfig(FP8KVConfig):
    """FP8 KV cache whose bytes the attention kernel reads directly (the reference allows ``scale="none"`` only;
    the paged kernel also reads per-head scales, ``"head"``, on the models it takes)."""

    technique: ClassVar[str] = "kv_fp8_fused"

    def __post_init__(self) -> None:
        super().__post_init__()
        if self.scale not in ("none", "head"):
            raise ConfigError("kv_fp8_fused supports scale='none' or 'head'; use kv_fp8 for per-token scales")

    def validate(self, adapter) -> None:
        """Refuses an attention implementation that does not read fp8 K/V (fused.py:39-49) and head dims beyond the
        dense kernel's 512 (its fp8 buffers)."""
        from .attention import accepts_fp8_kv

        super().validate(adapter)
        _dense_head_dim(self.technique, adapter, kv_in_model_dtype=False)
        _needs_kernel(self.technique, attn_implementation(adapter), accepts_fp8_kv, "fp8 K/V", "kv_fp8")


@dataclass(frozen=True)
class KIVIConfig(TechniqueConfig):
    """KIVI KV-cache quantization.

    Attributes:
        bits: Bits per quantized element (2, 4 or 8).
        group_size: Tokens per key group and channels per value group (32 in the paper).
        residual_length: Most recent tokens kept in full precision (a multiple of ``group_size``).
        layers: 1-indexed layers whose cache is quantized (empty: every layer).
        storage: ``"packed"``, ``"simulated"`` or ``None`` (as the reference; the paged cache is packed storage).
        headroom: Ring slots beyond ``residual_length`` for the uncommitted tokens of a cycle.
    """

    technique: ClassVar[str] = "kivi"
    #: Whether the configuration may use another storage than ``"simulated"``.
    packable: ClassVar[bool] = True
    bits: int = 2
    group_size: int = 32
    residual_length: int = 128
    layers: tuple[int, ...] = ()
    storage: str | None = None
    headroom: int = 256

    def __post_init__(self) -> None:
        _choice("bits", self.bits, KIVI_BITS)
        _positive("group_size", self.group_size)
        _positive("residual_length", self.residual_length)
        if self.residual_length % self.group_size:
            raise ConfigError(
                f"residual_length ({self.residual_length}) must be a multiple of group_size ({self.group_size})")
        _layers(self.layers)
        _positive("headroom", self.headroom)
        if self.storage is not None:
            _choice("storage", self.storage, ("packed", "simulated"))
            if not self.packable and self.storage != "simulated":
                raise ConfigError(f"{self.technique} supports only storage='simulated', got {self.storage!r}")

    def validate(self, adapter) -> None:
        """Refuses head dims the dense decode kernel does not take (up to 512, 256 on fp32 models): the packed
        record of the configurations the paged cache cannot hold, and the simulated storage, are read by it."""
        _dense_head_dim(self.technique, adapter, kv_in_model_dtype=True)

    def layer_kind(self, adapter) -> str:
        """Where this configuration's layers live on ``adapter``'s model: ``"paged"`` (the paged KIVI cache),
        ``"packed"`` (the reference's packed record and rings, techniques/kv_quant/packed.py:1-30: any bits, group,
        head dim and dtype) or ``"simulated"`` (dense buffers quantized in place, kivi.py:178-275)."""
        if self.storage == "simulated":
            return "simulated"
        return "paged" if kivi_paged_refusal(self, adapter) is None else "packed"

    @property
    def kivi_storage(self) -> str:
        """:attr:`storage`, else ``"packed"`` (``"simulated"`` for a configuration that is not :attr:`packable`)."""
        if self.storage is not None:
            return self.storage
        return "packed" if self.packable else "simulated"


@dataclass(frozen=True)
class FusedKIVIConfig(KIVIConfig):
    """KIVI whose packed codes the attention kernel reads directly (the reference keeps dense buffers beside the
    codes, so its only storage is ``"simulated"``; the paged cache holds the codes and the residual rings)."""

    technique: ClassVar[str] = "kivi_fused"
    packable: ClassVar[bool] = False

    def layer_kind(self, adapter) -> str:
        """``"paged"`` where the paged KIVI cache holds the layers, else ``"fused"``: dense buffers of the
        dequantized values with the reference's packed codes beside them (kv_kivi_fused/fused.py:104-250)."""
        return "paged" if kivi_paged_refusal(self, adapter) is None else "fused"

    def validate(self, adapter) -> None:
        """Refuses an attention implementation that does not read KIVI codes (kv_kivi_fused/fused.py:43-51)."""
        from .attention import accepts_packed_kv

        super().validate(adapter)
        _needs_kernel(self.technique, attn_implementation(adapter), lambda name: accepts_packed_kv(name, "kivi"),
                      "KIVI codes", "kivi")


@dataclass(frozen=True)
class QuestConfig(TechniqueConfig):
    """Quest: query-aware selection of cache pages at decode time.

    Attributes:
        page_size: Slots per page (a power of two, at least 16).
        token_budget: Entries every decoding query reads, the running page included.
        dense_layers: The first cache layers that attend densely.
        max_queries: Longest query restricted to the pages.
        layers: 1-indexed layers Quest acts on (empty: every layer).
        include_sliding: Also restrict sliding-window layers.
        first_page: Always select every row's first page (the "first and last pages" variant of Quest). The
            reference has no such rule (quest/technique.py:84-86 selects by score only), so it is off by default.
    """

    technique: ClassVar[str] = "quest"
    page_size: int = 16
    token_budget: int = 2048
    dense_layers: int = 2
    max_queries: int = 1
    layers: tuple[int, ...] = ()
    include_sliding: bool = False
    first_page: bool = False

    def __post_init__(self) -> None:
        if self.page_size < 16 or self.page_size & (self.page_size - 1):
            raise ConfigError(f"quest page_size must be a power of two of at least 16, got {self.page_size}")
        if self.token_budget < 2 * self.page_size:
            raise ConfigError(
                f"quest token_budget {self.token_budget} must hold at least two pages of {self.page_size} slots")
        if self.dense_layers < 0:
            raise ConfigError(f"quest dense_layers must be non-negative, got {self.dense_layers}")
        if self.max_queries < 1:
            raise ConfigError(f"quest max_queries must be positive, got {self.max_queries}")
        _layers(self.layers)

    @property
    def pages(self) -> int:
        """Committed pages a decoding query reads (the page budget minus the running page)."""
        return self.token_budget // self.page_size - 1

    def validate(self, adapter) -> None:
        """Refuses an attention implementation that does not read Quest pages (quest/technique.py:88-97) and head
        dims no Quest kernel takes: the paged kernels take bf16 models of head dim 64 / 128 / 256, the dense ones any
        dtype and any head dim that is a multiple of 8, up to 512 (256 on fp32 models)."""
        from .attention import accepts_packed_kv

        dim = head_dim_of(adapter)
        if dim is not None and dim % 8:
            raise ConfigError(f"{self.technique}: the MI355X kernels take head dims that are multiples of 8, the model "
                              f"has {dim}")
        _dense_head_dim(self.technique, adapter, kv_in_model_dtype=True)
        _needs_kernel(self.technique, attn_implementation(adapter), lambda name: accepts_packed_kv(name, "quest"),
                      "its pages", None)


# ---- techniques -----------------------------------------------------------------------------------------------

TECHNIQUES: Registry = Registry("technique")


def register_technique(cls):
    """Class decorator: registers a :class:`Technique` under its configuration's technique name."""
    TECHNIQUES.register(cls.config_class.technique, cls)
    return cls


def technique_for(config) -> Technique:
    """The technique of ``config`` (``ConfigError`` for an unregistered configuration type)."""
    technique = getattr(type(config), "technique", None)
    if technique is None:
        raise ConfigError(f"{type(config).__name__} is not a technique configuration")
    return TECHNIQUES.get_entry(technique)(config)


class Technique:
    """A registered technique: its configuration and the paged layer cache it makes."""

    config_class: ClassVar[type]
    #: The packed format the technique hands to attention ("kivi", "quest") or None.
    packed_format: ClassVar[str | None] = None

    def __init__(self, config) -> None:
        if not isinstance(config, self.config_class):
            raise ConfigError(f"{type(self).__name__} takes a {self.config_class.__name__}")
        self.config = config

    def covers(self, layer: int) -> bool:
        """Whether the technique acts on 1-indexed ``layer``."""
        return not self.config.layers or layer in self.config.layers

    def make_cache(self, **shape):
        raise NotImplementedError


@register_technique
class FP8KVTechnique(Technique):
    config_class = FP8KVConfig

    def make_cache(self, *, pages: int, kv_heads: int, head_dim: int, device, k_scale=None, v_scale=None, **_):
        """A paged fp8 cache (16-token pages); per-head scales for ``scale="head"``."""
        from .paged import PagedKVCache

        if self.config.scale in ("token", "tensor"):
            raise ConfigError(f"the paged fp8 cache stores per-head scales, not scale={self.config.scale!r}")
        if self.config.scale == "head" and (k_scale is None or v_scale is None):
            raise ConfigError("scale='head' needs per-head key and value scales (economize_amd.paged.head_scales)")
        return PagedKVCache.empty(pages, kv_heads, head_dim, self.config.dtype, device, k_scale, v_scale)


@register_technique
class FusedFP8KVTechnique(FP8KVTechnique):
    config_class = FusedFP8KVConfig


@register_technique
class KIVITechnique(Technique):
    config_class = KIVIConfig
    packed_format = "kivi"

    def make_cache(self, *, pages: int, batch: int, kv_heads: int, head_dim: int, device, **_):
        """A paged KIVI cache (32-token pages, residual ring of ``residual_length + headroom`` slots)."""
        from .kivi import PagedKIVICache

        c = self.config
        if c.storage == "simulated" and c.packable:
            raise ConfigError("the paged KIVI cache is packed storage, not storage='simulated'")
        return PagedKIVICache.empty(pages, batch, kv_heads, head_dim, c.bits, device, group=c.group_size,
                                    residual=c.residual_length, headroom=c.headroom)


@register_technique
class FusedKIVITechnique(KIVITechnique):
    config_class = FusedKIVIConfig


@register_technique
class QuestTechnique(Technique):
    config_class = QuestConfig
    packed_format = "quest"

    def covers(self, layer: int) -> bool:
        return layer > self.config.dense_layers and super().covers(layer)

    def make_cache(self, *, batch: int, kv_heads: int, head_dim: int, max_pages: int, device, **_):
        """Empty page bounds ``(kmin, kmax)`` bf16 ``[B, Hkv, max_pages, D]`` (the cache's keys themselves live in a
        paged fp8 or bf16 cache)."""
        shape = (batch, kv_heads, max_pages, head_dim)
        return (torch.zeros(shape, dtype=torch.bfloat16, device=device),
                torch.zeros(shape, dtype=torch.bfloat16, device=device))
