"""The Hugging Face drop-in of the compressed-KV path: ``apply`` attaches the techniques to a transformers causal LM
and :class:`EconomizeCache` is its ``past_key_values``, whose layers live in the paged MI355X caches.

Mirrors the reference's cache wrappers (techniques/_kv/wrapper.py:122-351: ``transform_update`` what is written for
new K/V, ``transform_read`` what attention sees, ``pass_begin`` / ``pass_end`` at the boundaries of an exact pass)
for the techniques of this path:

* ``FP8KVConfig`` / ``FusedFP8KVConfig``: K/V encoded to fp8 on write (``fp8_encode``, techniques/kv_quant/fp8.py:
  81-86 and 161-176). Where the paged kernels take the model (bf16, head dim 64 / 128 / 256) and the scale is none,
  static or per head, into a paged fp8 cache whose bytes attention reads on the paged kernel (kv_fp8_fused/fused.py:
  56-63 hands fp8 views over); otherwise into dense fp8 buffers (:class:`DenseFP8Layer`, also the per-token scales
  of fp8.py:95-97), handed to the dense kernel as fp8 views (fused) or decoded to the model's dtype (fp8.py:89-92).
  Static scales (``"tensor"``, and ``"head"`` per KV head) are calibrated at attach time (fp8.py:100-133).
* ``KIVIConfig`` / ``FusedKIVIConfig``: new tokens in the bf16 ring, the reference's schedule run at every pass
  boundary (the tokens a pass commits are quantized when it ends, kivi.py:191-243), attention on the fused KIVI
  kernel over codes and ring (kv_kivi_fused/fused.py:152-208). Configurations the paged KIVI cache cannot hold
  (8-bit codes, groups other than 32, other head dims or dtypes) keep the reference's packed record: codes and rings,
  no dense buffer (:class:`PackedKIVILayer`, kv_quant/packed.py:1-370), or, for ``FusedKIVIConfig``, codes beside
  dense buffers of the dequantized values (:class:`FusedKIVIDenseLayer`, kv_kivi_fused/fused.py:104-250); either
  way the kernel reads the codes. ``storage="simulated"`` keeps dense buffers quantized in place
  (:class:`SimulatedKIVILayer`, kivi.py:178-275).
* ``QuestConfig``: on a bf16 model of head dim 64 / 128 / 256 a paged bf16 cache whose page bounds live on the
  device (:class:`~economize_amd.quest.QuestState`: the append of a pass also computes the bounds of the pages
  committed before it, one launch); on other models dense buffers of the model's dtype (:class:`DenseQuestLayer`,
  bounds kept incrementally). ``done[b]`` = committed full pages before the pass; a decoding query of a covered layer
  reads the selected pages and the tail (quest/technique.py:116-259), and a layer whose attached pages no attention
  function read raises when it is written next (quest/technique.py:174-182).

A layer of no technique keeps dense K/V (transformers' ``DynamicLayer``) and attends on the dense kernel.

transformers calls the cache's ``update`` once per layer and pass, with no pass boundaries; a pass's boundary is
therefore taken at the next pass's first write of a layer: a layer's ``pass_begin`` runs when the layer is written
with a new frontier (its committed length grows), before the write, which is when the reference's ``pass_end`` of the
previous pass has taken effect for every later read.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from transformers.cache_utils import Cache, CacheLayerMixin, DynamicLayer

from .attention import MAX_QUERIES, NAME, PagedKV, install
from .errors import ConfigError, IncompatibleTechniquesError
from .fp8 import calibrate_kv_absmax, fp8_encode, static_scales
from .kivi import KIVI_PAGE, PagedKIVICache, kivi_append, kivi_commit, kivi_fake_quantize, kivi_quantize
from .packed import attach_packed, stand_in
from .paged import PAGE, PagedKVCache, paged_append
from .quest import QuestPages, QuestState, bounds_dtype, page_bounds
from .techniques import (FP8KVConfig, FusedFP8KVConfig, FusedKIVIConfig, KIVIConfig, QuestConfig, Technique,
                         attn_implementation, head_dim_of, technique_for)

__all__ = ["DenseFP8Layer", "DenseQuestLayer", "EconomizeCache", "EconomizedModel", "FusedKIVIDenseLayer", "KIVILayer",
           "PackedKIVILayer", "PagedLayer", "SimulatedKIVILayer", "apply"]


class _PagedBase(CacheLayerMixin):
    """The part every paged layer shares: rows of equal length (transformers' positions), a block table in which
    row ``b`` owns pages ``b * P .. b * P + P - 1``, the length written so far and the committed length (the
    frontier of the last pass)."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, capacity: int, page: int) -> None:
        super().__init__()
        self.capacity = int(capacity)
        self.page = page
        self.length = 0
        self.committed = 0
        self.model_dtype = torch.bfloat16
        self.table: torch.Tensor | None = None
        self._lens: dict[int, torch.Tensor] = {}

    def _allocate_table(self, batch: int, device: torch.device) -> int:
        per_row = -(-self.capacity // self.page)
        self.table = torch.arange(batch * per_row, dtype=torch.int32, device=device).view(batch, per_row)
        return batch * per_row

    def _seq_lens(self) -> torch.Tensor:
        lens = self._lens.get(self.length)
        if lens is None:
            self._lens = {self.length: torch.full((self.table.shape[0],), self.length, dtype=torch.int32,
                                                  device=self.table.device)}
            lens = self._lens[self.length]
        return lens

    def _check_room(self, tokens: int) -> None:
        if self.length + tokens > self.capacity:
            raise ConfigError(f"the cache holds {self.capacity} tokens per row; writing {tokens} more after "
                              f"{self.length} exceeds it (make the cache with a larger max_length)")

    def _stand_ins(self, key_states: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        batch, heads, _, dim = key_states.shape
        shape = (batch, heads, self.length, dim)
        return stand_in(shape, self.model_dtype, key_states.device), stand_in(shape, self.model_dtype,
                                                                              key_states.device)

    # ---- transformers' layer API -----------------------------------------------------------------------------------
    def get_seq_length(self) -> int:
        return self.length

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_max_length(self) -> int:
        return self.capacity

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if self.length > self.committed:
            self.pass_begin(self.length)
        key_states, value_states = self.transform_update(key_states, value_states)
        return self.transform_read(key_states, value_states)

    # ---- the cache-wrapper hooks -----------------------------------------------------------------------------------
    def pass_begin(self, frontier: int) -> None:
        """A new exact pass starts writing at ``frontier``: every token below it is committed."""
        self.committed = frontier

    def transform_update(self, key_states, value_states):
        raise NotImplementedError

    def transform_read(self, key_states, value_states):
        raise NotImplementedError

    def reset(self) -> None:
        self.length = self.committed = 0


class _UnreadCheck:
    """The reference's check that every attached page list was read (techniques/quest/technique.py:174-182): a Quest
    layer notes an attachment and its reading; a layer whose attachment no attention function read (another
    attention implementation, or a technique that copied the keys) raises when it is written next, so that Quest
    never decodes densely without a word."""

    def _init_unread(self, layer: int) -> None:
        self.layer_idx = layer
        self._unread = False

    def _attached(self) -> None:
        self._unread = True

    def _read(self, layer: int) -> None:
        self._unread = False

    def _check_read(self) -> None:
        if self._unread:
            self._unread = False
            raise IncompatibleTechniquesError(
                f"quest attached pages to cache layer {self.layer_idx} that no attention function read: run the model "
                "with attn_implementation='economize' (economize_amd.attention.install()) and let no technique copy "
                "the keys after quest")


class PagedLayer(_PagedBase, _UnreadCheck):
    """One layer in a paged fp8 or bf16 cache (16-token pages), optionally with Quest's page bounds, which live in a
    :class:`~economize_amd.quest.QuestState` on the device: the append of a pass also computes the bounds of the pages
    the previous passes committed (one launch, ``eco_paged_append_quest``), and ``done`` is a device tensor."""

    def __init__(self, capacity: int, cache_dtype: torch.dtype | None, quest: QuestConfig | None = None,
                 scales: tuple[torch.Tensor, torch.Tensor] | None = None, layer: int = 0, static: bool = False) -> None:
        super().__init__(capacity, PAGE)
        self.cache_dtype = cache_dtype  # None: the model's dtype (bf16)
        self.quest = quest
        self.scales = scales  # fp32 [Hkv] key and value scales of an fp8 cache, or None
        self.cache: PagedKVCache | None = None
        self.state: QuestState | None = None
        self._committed: dict[int, torch.Tensor] = {}
        self._write_width = 0
        self._init_unread(layer)
        # static: the written length, the committed lengths and the sequence lengths live on the device, and reads
        # hand over capacity-long stand-ins, so that a decode step has fixed shapes and can be captured in a graph
        self.static = static
        self._length_dev: torch.Tensor | None = None
        self._committed_dev: torch.Tensor | None = None
        self._lens_dev: torch.Tensor | None = None

    @property
    def bounds(self) -> tuple[torch.Tensor, torch.Tensor] | None:
        """Quest's ``(kmin, kmax)`` bf16 ``[B, Hkv, pages, D]``; pages below ``committed // page_size`` are valid."""
        return None if self.state is None else (self.state.kmin, self.state.kmax)

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        batch, heads, _, dim = key_states.shape
        self.model_dtype = key_states.dtype
        dtype = self.cache_dtype or torch.bfloat16
        pages = self._allocate_table(batch, key_states.device)
        k_scale = v_scale = None
        if self.scales is not None:
            k_scale, v_scale = (x.to(key_states.device, torch.float32).reshape(heads).contiguous() for x in self.scales)
        self.cache = PagedKVCache.empty(pages, heads, dim, dtype, key_states.device, k_scale, v_scale)
        q = self.quest
        if q is not None:
            self.state = QuestState(batch, heads, dim, max(1, self.capacity // q.page_size), q.page_size, q.pages,
                                    key_states.device, q.max_queries, q.first_page)
        if self.static:
            self._length_dev = torch.zeros(1, dtype=torch.int32, device=key_states.device)
            self._committed_dev = torch.zeros(batch, dtype=torch.int32, device=key_states.device)
            self._lens_dev = torch.zeros(batch, dtype=torch.int32, device=key_states.device)
        self.is_initialized = True

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return (self.capacity, 0) if self.static else (self.length + query_length, 0)

    def get_seq_length(self) -> int | torch.Tensor:
        """The tokens written; a static layer gives its device count (int32 ``[1]``), as transformers' static layers
        do, so that the positions and the causal mask transformers derives from it follow the device in a replayed
        graph."""
        if self.static and self._length_dev is not None:
            return self._length_dev.clone()
        return self.length

    def _committed_rows(self) -> torch.Tensor:
        lens = self._committed.get(self.committed)
        if lens is None:
            self._committed = {self.committed: torch.full((self.table.shape[0],), self.committed, dtype=torch.int32,
                                                          device=self.table.device)}
            lens = self._committed[self.committed]
        return lens

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        self._check_read()
        if self.static:
            return self._static_update(key_states, value_states)
        return super().update(key_states, value_states, *args, **kwargs)

    def _static_update(self, key_states: torch.Tensor, value_states: torch.Tensor
                       ) -> tuple[torch.Tensor, torch.Tensor]:
        """A pass of the static layer, every count on the device: the tokens written before it are committed, the
        new ones go to positions ``length ..`` (with Quest, the append also computes the bounds of the committed
        pages), and attention gets capacity-long stand-ins whose handle carries the device lengths. The host
        ``length`` counts eager passes only (a replayed graph advances the device one): callers pass position ids."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        batch, heads, tokens, dim = key_states.shape
        self._check_room(tokens)
        device = key_states.device
        self._committed_dev.copy_(self._length_dev.expand(batch))
        pos = torch.arange(tokens, dtype=torch.int32, device=device) + self._length_dev
        # a position past the capacity (a graph replayed too often) writes nothing instead of indexing past the table
        page_of = (pos // PAGE).clamp(max=self.table.shape[1] - 1).long()
        slots = torch.where(pos < self.capacity, self.table[:, page_of] * PAGE + pos % PAGE, -1)
        slots = slots.to(torch.int32).reshape(-1)
        k = key_states.transpose(1, 2).reshape(batch * tokens, heads, dim)
        v = value_states.transpose(1, 2).reshape(batch * tokens, heads, dim)
        if self.state is not None:
            self.state.append(self.cache, k, v, slots, self.table, self._committed_dev)
        else:
            paged_append(self.cache, k, v, slots)
        self._length_dev.add_(tokens)
        self._lens_dev.copy_(self._length_dev.expand(batch))
        self.committed, self.length, self._write_width = self.length, self.length + tokens, tokens
        pages = None
        q = self.quest
        if q is not None and tokens <= q.max_queries:
            pages = self.state.pages_handle(on_use=self._read, layer=self.layer_idx)
            self._attached()
        handle = PagedKV(self.cache, self.table, self._lens_dev, self.capacity, pages, self.model_dtype,
                         static=True)
        shape = (batch, heads, self.capacity, dim)
        keys = stand_in(shape, self.model_dtype, device)
        return attach_packed(keys, handle), stand_in(shape, self.model_dtype, device)

    def transform_update(self, key_states, value_states):
        """fp8_encode (or the bf16 rounding) of the new tokens into their pages, at positions ``length ..``; with
        Quest, the bounds of the pages committed since the last pass in the same launch."""
        batch, heads, tokens, dim = key_states.shape
        self._check_room(tokens)
        pos = torch.arange(self.length, self.length + tokens, device=key_states.device)
        slots = (self.table[:, pos // PAGE] * PAGE + pos % PAGE).to(torch.int32).reshape(-1)
        k = key_states.transpose(1, 2).reshape(batch * tokens, heads, dim)
        v = value_states.transpose(1, 2).reshape(batch * tokens, heads, dim)
        if self.state is not None:
            self.state.append(self.cache, k, v, slots, self.table, self._committed_rows())
        else:
            paged_append(self.cache, k, v, slots)
        self.length += tokens
        self._write_width = tokens
        return key_states, value_states

    def transform_read(self, key_states, value_states):
        """Stand-ins for the dense K/V with the paged handle attached; a decoding query of a Quest layer also gets
        the page bounds of the committed pages (attached only when ``max(done) > pages``, as the reference)."""
        pages = None
        q = self.quest
        if q is not None and self._write_width <= q.max_queries:
            done = min(self.committed // q.page_size, self.state.max_pages)
            if done > q.pages:
                pages = QuestPages(self.state.kmin, self.state.kmax, self.state.done, done, done, q.page_size, q.pages,
                                   max_queries=q.max_queries, on_use=self._read, layer=self.layer_idx,
                                   first_page=q.first_page)
                self._attached()
        handle = PagedKV(self.cache, self.table, self._seq_lens(), self.length, pages, self.model_dtype)
        keys, values = self._stand_ins(key_states)
        return attach_packed(keys, handle), values

    def reset(self) -> None:
        super().reset()
        self._unread = False
        if self.state is not None:
            self.state.reset()
        for t in (self._length_dev, self._committed_dev, self._lens_dev):
            if t is not None:
                t.zero_()


class DenseQuestLayer(CacheLayerMixin, _UnreadCheck):
    """Quest over dense ``[B, Hkv, capacity, D]`` K/V buffers of the model's dtype: the reference's own cache layout
    (runtime/cache.py:359-432) under its ``QuestCache`` (techniques/quest/technique.py:116-259), for the models the
    paged kernels do not take (fp16 / fp32, head dims other than 64 / 128 / 256). At a new pass every token before
    it is committed (``done = committed // page_size``); a decoding query (at most ``max_queries`` tokens) of a layer
    with more than ``pages`` committed pages gets the bounds of the committed pages (kept incrementally by
    ``eco_quest_dense_bounds``) attached to its keys, and attends over the selected pages and the tail on the dense
    decode kernel (``eco_quest_decode``)."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, capacity: int, config: QuestConfig, layer: int = 0) -> None:
        super().__init__()
        self.capacity = int(capacity)
        self.config = config
        self.length = self.committed = self.valid = 0
        self.buffers: tuple[torch.Tensor, torch.Tensor] | None = None
        self.bounds: tuple[torch.Tensor, torch.Tensor] | None = None
        self._done: dict[int, torch.Tensor] = {}
        self._init_unread(layer)

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        batch, heads, _, dim = key_states.shape
        device = key_states.device
        self.buffers = (torch.zeros(batch, heads, self.capacity, dim, dtype=key_states.dtype, device=device),
                        torch.zeros(batch, heads, self.capacity, value_states.shape[3], dtype=value_states.dtype,
                                    device=device))
        shape = (batch, heads, max(1, self.capacity // self.config.page_size), dim)
        dtype = bounds_dtype(key_states.dtype)
        self.bounds = (torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device))
        self.is_initialized = True

    def get_seq_length(self) -> int:
        return self.length

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_max_length(self) -> int:
        return self.capacity

    def _done_rows(self, done: int) -> torch.Tensor:
        rows = self._done.get(done)
        if rows is None:
            self._done = {done: torch.full((self.buffers[0].shape[0],), done, dtype=torch.int32,
                                           device=self.buffers[0].device)}
            rows = self._done[done]
        return rows

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self._check_read()
        if self.length > self.committed:
            self.committed = self.length  # pass_begin: everything written before this pass is committed
        tokens = key_states.shape[2]
        if self.length + tokens > self.capacity:
            raise ConfigError(f"the cache holds {self.capacity} tokens per row; writing {tokens} more after "
                              f"{self.length} exceeds it (make the cache with a larger max_length)")
        new = slice(self.length, self.length + tokens)
        self.buffers[0][:, :, new].copy_(key_states)
        self.buffers[1][:, :, new].copy_(value_states)
        self.length += tokens
        keys, values = (b[:, :, : self.length] for b in self.buffers)
        c = self.config
        done = self.committed // c.page_size
        if tokens > c.max_queries or done <= c.pages:
            return keys, values
        if self.valid < done:  # the bounds of the pages committed since the last refresh
            page_bounds(self.buffers[0], self.valid, done, c.page_size, out=self.bounds)
            self.valid = done
        pages = QuestPages(self.bounds[0], self.bounds[1], self._done_rows(done), done, done, c.page_size, c.pages,
                           max_queries=c.max_queries, on_use=self._read, layer=self.layer_idx,
                           first_page=c.first_page)
        self._attached()
        return attach_packed(keys, pages), values

    def reset(self) -> None:
        self.length = self.committed = self.valid = 0
        self._unread = False


class DenseFP8Layer(CacheLayerMixin):
    """One layer's K/V as fp8 codes in dense ``[B, Hkv, capacity, D]`` buffers (the reference's ``FP8Cache``,
    fp8.py:143-217): new K/V are encoded on write with the configuration's scale (none, per token, or the calibrated
    static scale per head); a read hands the fp8 buffers over as they are (``fused``: the economize kernel reads fp8
    K/V, kv_fp8_fused/fused.py:56-63) or decoded to the model's dtype as ``fp8_decode`` does (``codes * scale`` in
    fp32, then the model's dtype, fp8.py:89-92)."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, capacity: int, config: FP8KVConfig, fused: bool,
                 scales: tuple[torch.Tensor, torch.Tensor] | None = None) -> None:
        super().__init__()
        if fused and config.scale != "none":
            raise ConfigError("the dense fused fp8 cache takes scale='none' (kv_fp8_fused/fused.py:37-41)")
        self.capacity = int(capacity)
        self.config = config
        self.fused = fused
        self.scales = scales
        self.length = 0
        self.model_dtype = torch.bfloat16
        self.codes: tuple[torch.Tensor, torch.Tensor] | None = None
        self.token_scales: tuple[torch.Tensor, torch.Tensor] | None = None
        self.head_scales: tuple[torch.Tensor, torch.Tensor] | None = None

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        batch, heads, _, dim = key_states.shape
        device = key_states.device
        self.model_dtype = key_states.dtype
        self.codes = tuple(torch.zeros(batch, heads, self.capacity, dim, dtype=self.config.dtype, device=device)
                           for _ in range(2))
        if self.config.scale == "token":
            self.token_scales = tuple(torch.ones(batch, heads, self.capacity, dtype=torch.float32, device=device)
                                      for _ in range(2))
        elif self.config.scale in ("tensor", "head"):
            if self.scales is None:
                raise ConfigError(f"scale={self.config.scale!r} needs calibrated scales (apply(..., calibration=))")
            self.head_scales = tuple(x.to(device, torch.float32).reshape(heads).contiguous() for x in self.scales)
        self.is_initialized = True

    def get_seq_length(self) -> int:
        return self.length

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_max_length(self) -> int:
        return self.capacity

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        tokens = key_states.shape[2]
        if self.length + tokens > self.capacity:
            raise ConfigError(f"the cache holds {self.capacity} tokens per row; writing {tokens} more after "
                              f"{self.length} exceeds it (make the cache with a larger max_length)")
        new = slice(self.length, self.length + tokens)
        for i, states in enumerate((key_states, value_states)):
            states = states if states.stride(-1) == 1 else states.contiguous()
            fp8_encode(states, self.config.dtype, self.codes[i][:, :, new],
                       None if self.head_scales is None else self.head_scales[i],
                       None if self.token_scales is None else self.token_scales[i][:, :, new])
        self.length += tokens
        keys, values = (c[:, :, : self.length] for c in self.codes)
        if self.fused:
            return keys, values
        return self._decoded(keys, 0), self._decoded(values, 1)

    def _decoded(self, codes: torch.Tensor, i: int) -> torch.Tensor:
        work = codes.float()
        if self.token_scales is not None:
            work = work * self.token_scales[i][:, :, : self.length, None]
        elif self.head_scales is not None:
            work = work * self.head_scales[i].view(1, -1, 1, 1)
        return work.to(self.model_dtype)

    def reset(self) -> None:
        self.length = 0


class KIVILayer(_PagedBase):
    """One layer in the paged KIVI cache (32-token pages) with its bf16 ring of ``residual + headroom`` slots.

    A pass of at most ``headroom`` tokens writes them to the ring; what it commits is quantized from the ring when
    the next pass begins (the reference's ``kivi_commit`` at a pass boundary). A longer pass (a prompt) cannot leave
    its tokens in the ring: what the schedule quantizes at its end is quantized as it writes, from the ring's
    unquantized past and the pass's own K/V, and the pass itself reads its tokens as it computed them (the dense view
    its attention falls back to, such a query being longer than the kernels take).
    """

    def __init__(self, capacity: int, config: KIVIConfig) -> None:
        super().__init__(capacity, KIVI_PAGE)
        if config.headroom < MAX_QUERIES:
            raise ConfigError(f"the paged KIVI layer needs headroom >= {MAX_QUERIES} (a decoding pass's tokens stay in "
                              f"the ring until the pass ends), got {config.headroom}")
        self.config = config
        self.cache: PagedKIVICache | None = None
        self.kq = 0  # quantized keys / values of every row (the device counts' host mirror)
        self.vq = 0
        self._current: tuple[torch.Tensor, torch.Tensor] | None = None

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        batch, heads, _, dim = key_states.shape
        if key_states.dtype != torch.bfloat16:
            raise ConfigError(f"the paged KIVI cache takes a bf16 model, not {key_states.dtype}")
        self.model_dtype = key_states.dtype
        pages = self._allocate_table(batch, key_states.device)
        c = self.config
        self.cache = PagedKIVICache.empty(pages, batch, heads, dim, c.bits, key_states.device, group=c.group_size,
                                          residual=c.residual_length, headroom=c.headroom)
        self.is_initialized = True

    def _schedule(self, committed: int) -> tuple[int, int]:
        r = self.config.residual_length
        return max(self.kq, (committed // r) * r), max(self.vq, committed - r)

    def pass_begin(self, frontier: int) -> None:
        """The previous pass ended: quantize what it committed (kivi.py:230-243), from the ring."""
        if frontier > self.committed:
            batch = self.table.shape[0]
            committed = torch.full((batch,), frontier, dtype=torch.int32, device=self.table.device)
            kivi_commit(self.cache, self.table, committed, frontier - self.committed)
            self.kq, self.vq = self._schedule(frontier)
        super().pass_begin(frontier)

    def _quantize_pass(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Quantize what the schedule quantizes at the end of this long pass, from the ring's past tokens that are
        not quantized yet (below the pass) and the pass's own K/V."""
        from .kivi import kivi_gather

        batch, heads, tokens, dim = key_states.shape
        start = self.length
        kq, vq = self._schedule(start + tokens)
        lo = min(self.kq, self.vq)
        k_src, v_src = key_states, value_states
        if lo < start:  # at most residual + headroom tokens of the past, all in the ring
            past_k, past_v = kivi_gather(self.cache, self.table, start, torch.bfloat16)
            k_src = torch.cat([past_k[:, :, lo:], key_states], dim=2)
            v_src = torch.cat([past_v[:, :, lo:], value_states], dim=2)
        k_src, v_src = k_src.contiguous(), v_src.contiguous()
        device = key_states.device

        def rows(x: int) -> torch.Tensor:
            return torch.full((batch,), x, dtype=torch.int32, device=device)

        if kq > self.kq:
            kivi_quantize(self.cache, self.table, k_src, "k", rows(self.kq), rows(kq), kq - self.kq, source_start=lo)
        if vq > self.vq:
            kivi_quantize(self.cache, self.table, v_src, "v", rows(self.vq), rows(vq), vq - self.vq, source_start=lo)
        self.kq, self.vq = kq, vq
        self.committed = start + tokens  # this pass's boundary is done

    def transform_update(self, key_states, value_states):
        """The new tokens into the ring (the last ``ring`` of a longer pass); a pass longer than the headroom is
        quantized as it writes (:meth:`_quantize_pass`)."""
        batch, heads, tokens, dim = key_states.shape
        self._check_room(tokens)
        start = self.length
        device = key_states.device
        ring = self.cache.ring
        self._current = None
        if tokens > self.config.headroom:
            self._quantize_pass(key_states, value_states)
            self._current = (key_states, value_states)
        first = max(0, tokens - ring)
        width = tokens - first
        rows = torch.arange(batch, dtype=torch.int32, device=device).repeat_interleave(width)
        pos = torch.arange(start + first, start + tokens, dtype=torch.int32, device=device).repeat(batch)
        kivi_append(self.cache, key_states[:, :, first:].transpose(1, 2).reshape(batch * width, heads, dim),
                    value_states[:, :, first:].transpose(1, 2).reshape(batch * width, heads, dim), rows, pos)
        self.length += tokens
        self.cache.keys_quantized.fill_(self.kq)
        self.cache.values_quantized.fill_(self.vq)
        return key_states, value_states

    def transform_read(self, key_states, value_states):
        handle = PagedKV(self.cache, self.table, self._seq_lens(), self.length, None, self.model_dtype,
                         self._current)
        keys, values = self._stand_ins(key_states)
        return attach_packed(keys, handle), values

    def reset(self) -> None:
        super().reset()
        self.kq = self.vq = 0


class SimulatedKIVILayer(CacheLayerMixin):
    """KIVI's simulated storage (the reference's ``KIVICache``, kivi.py:178-275): dense ``[B, Hkv, capacity, D]``
    buffers of the model's dtype whose committed entries are quantized in place when the next pass begins (keys below
    ``(c // R) * R``, values below ``c - R``) by ``eco_kivi_fake_quantize``; attention reads the buffers (the dense
    kernel). The values held are the ones the fused kernels dequantize, so any bits, group size and head dim run with
    the paged technique's results, at the dense cache's size."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, capacity: int, config: KIVIConfig) -> None:
        super().__init__()
        self.capacity = int(capacity)
        self.config = config
        self.length = self.committed = self.kq = self.vq = 0
        self.buffers: tuple[torch.Tensor, torch.Tensor] | None = None

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        batch, heads, _, dim = key_states.shape
        self.buffers = tuple(torch.zeros(batch, heads, self.capacity, dim, dtype=key_states.dtype,
                                         device=key_states.device) for _ in range(2))
        self.is_initialized = True

    def get_seq_length(self) -> int:
        return self.length

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_max_length(self) -> int:
        return self.capacity

    def pass_begin(self, frontier: int) -> None:
        """Quantize what the schedule quantizes once ``frontier`` tokens are committed (kivi.py:230-243)."""
        c = self.config
        k_to, v_to = max(self.kq, (frontier // c.residual_length) * c.residual_length), max(self.vq, frontier -
                                                                                            c.residual_length)
        if k_to > self.kq:
            kivi_fake_quantize(self.buffers[0], self.kq, k_to, c.bits, c.group_size, "k")
        if v_to > self.vq:
            kivi_fake_quantize(self.buffers[1], self.vq, v_to, c.bits, c.group_size, "v")
        self.kq, self.vq, self.committed = k_to, v_to, frontier

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if self.length > self.committed:
            self.pass_begin(self.length)
        tokens = key_states.shape[2]
        if self.length + tokens > self.capacity:
            raise ConfigError(f"the cache holds {self.capacity} tokens per row; writing {tokens} more after "
                              f"{self.length} exceeds it (make the cache with a larger max_length)")
        new = slice(self.length, self.length + tokens)
        self.buffers[0][:, :, new].copy_(key_states)
        self.buffers[1][:, :, new].copy_(value_states)
        self.length += tokens
        return tuple(b[:, :, : self.length] for b in self.buffers)

    def reset(self) -> None:
        self.length = self.committed = self.kq = self.vq = 0


class FusedKIVIDenseLayer(SimulatedKIVILayer):
    """``FusedKIVIConfig`` where the paged KIVI cache cannot hold the layer (the reference's ``FusedKIVICache``,
    kv_kivi_fused/fused.py:104-250): the simulated storage's dense buffers, plus the codes, fp16 scales and zero
    points of every quantized entry in the reference's ``KIVIPacked`` layout (:class:`~economize_amd.kivi_packed.
    KIVIPackedStore`). A pass boundary quantizes the committed entries once, writing the codes and the dequantized
    values into the buffers (``eco_kivi_pack_quantize``); attention gets the buffers with the record attached, and the
    kernel reads the quantized prefix as codes (``eco_kivi_packed_decode``), the rest from the buffers. A scale or
    zero point beyond fp16 stops the attachment for the rest of the generation (its fp16 copy would not give the
    buffer's values), as the reference stops it (fused.py:132-141); attention then reads the buffers."""

    def __init__(self, capacity: int, config: KIVIConfig) -> None:
        super().__init__(capacity, config)
        self.store = None
        self.packable = True

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        from .kivi_packed import KIVIPackedStore

        super().lazy_initialization(key_states, value_states)
        batch, heads, _, dim = key_states.shape
        c = self.config
        self.store = KIVIPackedStore(batch, heads, self.capacity, dim, value_states.shape[3], c.bits, c.group_size,
                                     key_states.device)

    def pass_begin(self, frontier: int) -> None:
        """Quantize what the schedule quantizes once ``frontier`` tokens are committed (kivi.py:230-243), into the
        record and the buffers."""
        c = self.config
        k_to = max(self.kq, (frontier // c.residual_length) * c.residual_length)
        v_to = max(self.vq, frontier - c.residual_length)
        store = self.store
        batch = self.buffers[0].shape[0]
        device = self.buffers[0].device

        def rows(x: int) -> torch.Tensor:
            return torch.full((batch,), x, dtype=torch.int32, device=device)

        if k_to > self.kq:
            store.quantize(self.buffers[0], "k", rows(self.kq), rows(k_to), k_to - self.kq, write_back=True)
            store.keys_quantized.fill_(k_to)
        if v_to > self.vq:
            store.quantize(self.buffers[1], "v", rows(self.vq), rows(v_to), v_to - self.vq, write_back=True)
            store.values_quantized.fill_(v_to)
        if (k_to > self.kq or v_to > self.vq) and self.packable and int(store.overflow.item()):
            self.packable = False
        self.kq, self.vq, self.committed = k_to, v_to, frontier

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        keys, values = super().update(key_states, value_states, *args, **kwargs)
        if not self.packable or (self.kq == 0 and self.vq == 0):
            return keys, values
        return attach_packed(keys, self.store.record(self.length)), values

    def reset(self) -> None:
        super().reset()
        self.packable = True
        if self.store is not None:
            self.store.keys_quantized.zero_()
            self.store.values_quantized.zero_()
            self.store.overflow.zero_()


class PackedKIVILayer(CacheLayerMixin):
    """``KIVIConfig``'s packed storage where the paged KIVI cache cannot hold the layer (the reference's
    ``PackedKIVICache``, techniques/kv_quant/packed.py:1-370; any bits, group, head dim and dtype): no dense buffer,
    only the codes, fp16 scales and zero points of the quantized entries (:class:`~economize_amd.kivi_packed.
    KIVIPackedStore`) and two rings of ``residual_length + headroom`` slots in the model's dtype holding the entries
    not quantized yet (slot ``s`` at ``s % ring``).

    A pass of at most ``headroom`` tokens writes them to the rings and attends through zero-memory stand-ins carrying
    the packed record (``eco_kivi_packed_decode`` reads the codes and the rings); what it commits is quantized from
    the rings when the next pass begins. A longer pass (a prompt) gets a dense copy (``eco_kivi_packed_gather``) with
    its tokens written in, quantizes what its end commits from that copy and keeps only its last ``ring`` tokens in
    the rings. Attention paths that do not read codes get the dense copy (``materialize``).

    Raises:
        ConfigError: A pass would overwrite ring entries not quantized yet (raise ``headroom``), or a scale or zero
            point lies beyond fp16 (use ``storage="simulated"``), as the reference refuses both (packed.py:175-188).
    """

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, capacity: int, config: KIVIConfig) -> None:
        super().__init__()
        self.capacity = int(capacity)
        self.config = config
        self.ring = max(1, min(config.residual_length + config.headroom, self.capacity - 1))
        self.length = self.committed = self.kq = self.vq = 0
        self.store = None
        self.rings: tuple[torch.Tensor, torch.Tensor] | None = None

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        from .kivi_packed import KIVIPackedStore

        batch, heads, _, dim = key_states.shape
        c = self.config
        self.store = KIVIPackedStore(batch, heads, self.capacity, dim, value_states.shape[3], c.bits, c.group_size,
                                     key_states.device)
        self.rings = tuple(torch.zeros(batch, heads, self.ring + 1, x.shape[3], dtype=x.dtype, device=x.device)
                           for x in (key_states, value_states))
        self.is_initialized = True

    def get_seq_length(self) -> int:
        return self.length

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_max_length(self) -> int:
        return self.capacity

    def allocated_bytes(self) -> int:
        """Bytes the layer holds on the device (codes, scales, zero points, counts and rings)."""
        tensors = [self.store.key_codes, self.store.key_scale, self.store.key_zero, self.store.value_codes,
                   self.store.value_scale, self.store.value_zero, *self.rings]
        return sum(t.numel() * t.element_size() for t in tensors)

    def _schedule(self, committed: int) -> tuple[int, int]:
        r = self.config.residual_length
        return max(self.kq, (committed // r) * r), max(self.vq, committed - r)

    def _quantize(self, keys: torch.Tensor, values: torch.Tensor, k_to: int, v_to: int, ring: int) -> None:
        """Keys ``[kq, k_to)`` and values ``[vq, v_to)`` of every row from ``keys`` / ``values`` (the rings, or a
        dense copy with ``ring`` 0) into the record; refuses scales beyond fp16."""
        store = self.store
        batch = keys.shape[0]
        device = keys.device

        def rows(x: int) -> torch.Tensor:
            return torch.full((batch,), x, dtype=torch.int32, device=device)

        if k_to > self.kq:
            store.quantize(keys, "k", rows(self.kq), rows(k_to), k_to - self.kq, ring=ring)
            store.keys_quantized.fill_(k_to)
        if v_to > self.vq:
            store.quantize(values, "v", rows(self.vq), rows(v_to), v_to - self.vq, ring=ring)
            store.values_quantized.fill_(v_to)
        if (k_to > self.kq or v_to > self.vq) and int(store.overflow.item()):
            store.overflow.zero_()
            raise ConfigError("a KIVI scale or zero point exceeds the fp16 range of the packed storage; use "
                              "storage='simulated'")
        self.kq, self.vq = k_to, v_to

    def pass_begin(self, frontier: int) -> None:
        """Quantize what the schedule quantizes once ``frontier`` tokens are committed (kivi.py:230-243), from the
        rings."""
        k_to, v_to = self._schedule(frontier)
        self._quantize(self.rings[0], self.rings[1], k_to, v_to, self.ring)
        self.committed = frontier

    def _write_rings(self, keys: torch.Tensor, values: torch.Tensor, start: int) -> None:
        tokens = keys.shape[2]
        if start + tokens - min(self.kq, self.vq) > self.ring:
            raise ConfigError(f"a pass wrote more than the packed KIVI ring holds ({self.ring} slots = residual_length "
                              "+ headroom) and would overwrite entries not quantized yet: increase headroom or use "
                              "storage='simulated'")
        slots = torch.arange(start, start + tokens, device=keys.device) % self.ring
        self.rings[0].index_copy_(2, slots, keys.to(self.rings[0].dtype))
        self.rings[1].index_copy_(2, slots, values.to(self.rings[1].dtype))

    def _dense(self, length: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.store.materialize(self.rings[0], self.rings[1], self.ring, length)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if self.length > self.committed:
            self.pass_begin(self.length)
        tokens = key_states.shape[2]
        start = self.length
        if start + tokens > self.capacity:
            raise ConfigError(f"the cache holds {self.capacity} tokens per row; writing {tokens} more after {start} "
                              "exceeds it (make the cache with a larger max_length)")
        if tokens > self.config.headroom:  # a prompt: a dense copy, what its end commits packed from it
            old_k, old_v = self._dense(start)
            keys = torch.cat([old_k, key_states.to(old_k.dtype)], dim=2).contiguous()
            values = torch.cat([old_v, value_states.to(old_v.dtype)], dim=2).contiguous()
            end = start + tokens
            k_to, v_to = self._schedule(end)
            self._quantize(keys, values, k_to, v_to, 0)
            first = max(0, tokens - self.ring)
            self._write_rings(key_states[:, :, first:], value_states[:, :, first:], start + first)
            self.length = self.committed = end
            return keys, values
        self._write_rings(key_states, value_states, start)
        self.length += tokens
        length = self.length
        record = self.store.record(length, key_ring=self.rings[0], value_ring=self.rings[1], ring=self.ring,
                                   materialize=lambda: self._dense(length))
        batch, heads, _, dim = key_states.shape
        keys = attach_packed(stand_in((batch, heads, length, dim), key_states.dtype, key_states.device), record)
        values = stand_in((batch, heads, length, value_states.shape[3]), value_states.dtype, value_states.device)
        return keys, values

    def reset(self) -> None:
        self.length = self.committed = self.kq = self.vq = 0
        if self.store is not None:
            self.store.keys_quantized.zero_()
            self.store.values_quantized.zero_()
            self.store.overflow.zero_()


class EconomizeCache(Cache):
    """transformers ``past_key_values`` whose layers are the techniques' paged caches (dense ``DynamicLayer`` for a
    layer no technique covers)."""

    def __init__(self, layers: list[CacheLayerMixin]) -> None:
        super().__init__(layers=layers)

    def check_flags(self) -> None:
        """The reference's pass-boundary refusal of KIVI scales beyond fp16 (packed.py:175-188), for every layer."""
        for layer in self.layers:
            if isinstance(layer, KIVILayer) and layer.cache is not None:
                layer.cache.check_flags()


@dataclass
class EconomizedModel:
    """A transformers causal LM with the compressed-KV techniques attached (the reference's ``apply`` result,
    core/model.py:330-386, limited to this path): :meth:`make_cache` builds the ``past_key_values`` that hold its
    layers in the techniques' paged caches.

    Attributes:
        model: The transformers model (its attention implementation set to ``"economize"``).
        techniques: The attached techniques, in attach order.
    """

    model: torch.nn.Module
    techniques: list[Technique] = field(default_factory=list)
    #: Calibrated fp8 scales by 0-indexed layer: fp32 ``[Hkv]`` key and value scales (a static ``"tensor"`` scale
    #: repeated over the heads).
    scales: dict[int, tuple[torch.Tensor, torch.Tensor]] = field(default_factory=dict)

    def technique_of(self, layer: int) -> Technique | None:
        """The technique covering 1-indexed ``layer`` (at most one per layer)."""
        for technique in self.techniques:
            if technique.covers(layer):
                return technique
        return None

    def paged_fp8(self, config: FP8KVConfig) -> bool:
        """Whether ``config``'s layers live in the paged fp8 cache: the paged kernels take the model (bf16 or fp16,
        head dim 64 / 128 / 256) and the scale is one they read (none, or static per head); else dense fp8 buffers."""
        dtype = next(self.model.parameters()).dtype
        return dtype in (torch.bfloat16, torch.float16) and head_dim_of(self.model) in (64, 128, 256) and \
            config.scale != "token"

    def paged_quest(self) -> bool:
        """Whether Quest layers live in the paged bf16 cache (a bf16 model of head dim 64 / 128 / 256, which the paged
        kernels take); else in dense buffers of the model's dtype (:class:`DenseQuestLayer`)."""
        dtype = next(self.model.parameters()).dtype
        return dtype == torch.bfloat16 and head_dim_of(self.model) in (64, 128, 256)

    def make_cache(self, max_length: int, static: bool = False) -> EconomizeCache:
        """A cache for generations of up to ``max_length`` tokens per row (prompt included).

        ``static``: every layer in a paged cache whose lengths live on the device and whose reads have fixed shapes
        (:class:`PagedLayer` with ``static=True``), so that a decoding step, ``model(input_ids=..., position_ids=...,
        past_key_values=cache)`` with position ids from a device buffer, can be captured in a HIP graph and replayed;
        layers without a technique keep bf16 pages. It takes a bf16 model of head dim 64 / 128 / 256 and the fp8
        (none or per-head scale) and Quest techniques.
        """
        config = self.model.config
        layers: list[CacheLayerMixin] = []
        if static:
            dtype = next(self.model.parameters()).dtype
            if dtype != torch.bfloat16 or head_dim_of(self.model) not in (64, 128, 256):
                raise ConfigError("a static cache takes a bf16 model of head dim 64, 128 or 256")
        for index in range(config.num_hidden_layers):
            technique = self.technique_of(index + 1)
            cfg = technique.config if technique is not None else None
            if static:
                if isinstance(cfg, KIVIConfig) or (isinstance(cfg, FP8KVConfig) and not self.paged_fp8(cfg)):
                    raise ConfigError(f"a static cache holds layers of no technique, paged fp8 and Quest, not "
                                      f"{type(cfg).__name__} on layer {index + 1}")
                fp8 = cfg.dtype if isinstance(cfg, FP8KVConfig) else None
                quest = cfg if isinstance(cfg, QuestConfig) else None
                layers.append(PagedLayer(max_length, fp8, quest, scales=self.scales.get(index), layer=index,
                                         static=True))
                continue
            if isinstance(cfg, KIVIConfig):
                kind = cfg.layer_kind(self.model)
                layer_class = {"paged": KIVILayer, "packed": PackedKIVILayer, "fused": FusedKIVIDenseLayer,
                               "simulated": SimulatedKIVILayer}[kind]
                layers.append(layer_class(max_length, cfg))
            elif isinstance(cfg, FP8KVConfig) and self.paged_fp8(cfg):
                layers.append(PagedLayer(max_length, cfg.dtype, scales=self.scales.get(index)))
            elif isinstance(cfg, FP8KVConfig):
                layers.append(DenseFP8Layer(max_length, cfg, isinstance(cfg, FusedFP8KVConfig),
                                            self.scales.get(index)))
            elif isinstance(cfg, QuestConfig) and self.paged_quest():
                layers.append(PagedLayer(max_length, None, cfg, layer=index))
            elif isinstance(cfg, QuestConfig):
                layers.append(DenseQuestLayer(max_length, cfg, layer=index))
            else:
                layers.append(DynamicLayer())
        return EconomizeCache(layers)

    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, **kwargs) -> torch.Tensor:
        """transformers' ``generate`` with a fresh :class:`EconomizeCache` (greedy unless ``kwargs`` say otherwise)."""
        cache = self.make_cache(input_ids.shape[1] + max_new_tokens)
        kwargs.setdefault("do_sample", False)
        return self.model.generate(input_ids, past_key_values=cache, max_new_tokens=max_new_tokens, **kwargs)


def apply(model: torch.nn.Module, *configs, calibration=None) -> EconomizedModel:
    """Attach the techniques of ``configs`` to a transformers causal LM (core/model.py:330-356): registers the
    ``"economize"`` kernel (:func:`~economize_amd.attention.install`), selects it as the model's attention
    implementation, validates every configuration against the model before anything attaches
    (``config.validate(model)``), refuses two techniques on one layer, and calibrates the static fp8 scales of
    ``scale="tensor"`` / ``"head"`` on ``calibration`` (token batches; fp8.py:100-133).

    Raises:
        ConfigError: A configuration the MI355X path cannot run on this model, or static fp8 scales without
            calibration batches.
        IncompatibleTechniquesError: Two techniques cover one layer, or a technique twice.
    """
    install()
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation(NAME)
    else:
        model.config._attn_implementation = NAME
    if attn_implementation(model) != NAME:
        raise ConfigError(f"could not select the {NAME!r} attention implementation on {type(model).__name__}")
    if head_dim_of(model) is None:
        raise ConfigError(f"{type(model).__name__} has no attention head dimension in its config")
    techniques: list[Technique] = []
    for config in configs:
        if any(type(t.config) is type(config) for t in techniques):
            raise IncompatibleTechniquesError(f"{config.technique} is applied twice")
        config.validate(model)
        techniques.append(technique_for(config))
    for layer in range(1, model.config.num_hidden_layers + 1):
        covering = [t.config.technique for t in techniques if t.covers(layer)]
        if len(covering) > 1:
            raise IncompatibleTechniquesError(f"layer {layer} is covered by {covering}; one KV technique per layer")
    result = EconomizedModel(model, techniques)
    for technique in techniques:
        config = technique.config
        if not isinstance(config, FP8KVConfig):
            continue
        if isinstance(config, FusedFP8KVConfig) and config.scale == "head" and not result.paged_fp8(config):
            raise ConfigError("kv_fp8_fused with scale='head' needs the paged fp8 cache (a bf16 model of head dim "
                              "64, 128 or 256); use kv_fp8 on this model")
        if config.scale not in ("tensor", "head"):
            continue
        if calibration is None:
            raise ConfigError(f"scale={config.scale!r} is calibrated at attach time: pass calibration batches to "
                              "apply(model, ..., calibration=...)")
        keys, values = calibrate_kv_absmax(model, calibration, per_head=config.scale == "head")
        kv_heads = getattr(model.config, "num_key_value_heads", None) or model.config.num_attention_heads
        for index in range(model.config.num_hidden_layers):
            if technique.covers(index + 1):
                k, v = (static_scales(x[index], config.dtype).reshape(-1).expand(kv_heads).contiguous()
                        for x in (keys, values))
                result.scales[index] = (k, v)
    return result
