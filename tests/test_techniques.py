"""Host-side configuration, the technique registry and the ``"economize"`` attention registration, on the CPU.

Mirrors the reference's configuration tests: tests/techniques/test_quest.py:300-312 (QuestConfig validation and the
JSON round trip), tests/techniques/test_kv_kivi_packed.py:52-61 and :186-189 (KIVI storage and headroom),
tests/techniques/test_kv_fp8_fused.py:41-44 (fused fp8 refuses scales and unknown formats).
"""

from __future__ import annotations

import json

import pytest
import torch

from economize_amd.attention import (
    ATTENTION_KERNELS, PagedKV, accepts_fp8_kv, accepts_packed_kv, economize_attention_forward,
)
from economize_amd.errors import ConfigError, IncompatibleTechniquesError
from economize_amd.paged import PagedKVCache
from economize_amd.techniques import (
    TECHNIQUES, FP8KVConfig, FusedFP8KVConfig, FusedKIVIConfig, KIVIConfig, QuestConfig, Registry,
    register_technique, technique_for,
)


def test_quest_config_validation() -> None:
    for fields, match in (
        ({"page_size": 8}, "power of two"),
        ({"page_size": 24}, "power of two"),
        ({"token_budget": 16}, "two pages"),
        ({"dense_layers": -1}, "non-negative"),
        ({"max_queries": 0}, "positive"),
        ({"layers": (0,)}, "1-indexed"),
        ({"layers": [3]}, "tuple"),
    ):
        with pytest.raises(ConfigError, match=match):
            QuestConfig(**fields)
    assert QuestConfig().pages == 127
    assert QuestConfig(page_size=16, token_budget=48).pages == 2
    assert QuestConfig(page_size=64, token_budget=4096).pages == 63
    config = QuestConfig(token_budget=48, layers=(3, 4))
    assert QuestConfig.from_dict(json.loads(json.dumps(config.to_dict()))) == config


def test_kivi_config_validation() -> None:
    for fields, match in (
        ({"bits": 3}, "bits"),
        ({"group_size": 0}, "group_size"),
        ({"residual_length": 100}, "multiple of group_size"),
        ({"headroom": 0}, "headroom"),
        ({"storage": "paged"}, "storage"),
        ({"group_size": True}, "group_size"),
    ):
        with pytest.raises(ConfigError, match=match):
            KIVIConfig(**fields)
    assert KIVIConfig().kivi_storage == "packed"
    assert KIVIConfig(storage="simulated").kivi_storage == "simulated"
    with pytest.raises(ConfigError):
        FusedKIVIConfig(storage="packed")
    assert FusedKIVIConfig().kivi_storage == "simulated"
    config = KIVIConfig(bits=4, residual_length=64, layers=(1, 2))
    assert KIVIConfig.from_dict(json.loads(json.dumps(config.to_dict()))) == config
    with pytest.raises(ConfigError, match="unknown"):
        KIVIConfig.from_dict({"bits": 2, "window": 3})


def test_fp8_config_validation() -> None:
    with pytest.raises(ConfigError):
        FusedFP8KVConfig(scale="token")
    with pytest.raises(ConfigError):
        FusedFP8KVConfig(format="e3m4")
    with pytest.raises(ConfigError):
        FP8KVConfig(scale="channel")
    assert FP8KVConfig(format="e5m2").dtype == torch.float8_e5m2
    assert FusedFP8KVConfig(scale="head").dtype == torch.float8_e4m3fn


def test_techniques_are_registered_by_name() -> None:
    assert TECHNIQUES.names() == ["kivi", "kivi_fused", "kv_fp8", "kv_fp8_fused", "quest"]
    for config in (FP8KVConfig(), FusedFP8KVConfig(), KIVIConfig(), FusedKIVIConfig(), QuestConfig()):
        technique = technique_for(config)
        assert technique.config is config
        assert type(technique).config_class is type(config)
    with pytest.raises(ConfigError, match="already registered"):
        register_technique(type(technique_for(QuestConfig())))
    with pytest.raises(ConfigError, match="not a technique"):
        technique_for(object())
    with pytest.raises(ConfigError, match="unknown"):
        Registry("technique").get_entry("h2o")


def test_quest_covers_layers_above_the_dense_ones() -> None:
    quest = technique_for(QuestConfig(dense_layers=2))
    assert [layer for layer in range(1, 7) if quest.covers(layer)] == [3, 4, 5, 6]
    quest = technique_for(QuestConfig(dense_layers=2, layers=(1, 4)))
    assert [layer for layer in range(1, 7) if quest.covers(layer)] == [4]
    kivi = technique_for(KIVIConfig(layers=(2,)))
    assert [layer for layer in range(1, 4) if kivi.covers(layer)] == [2]


def test_economize_kernel_is_registered() -> None:
    assert "economize" in ATTENTION_KERNELS.names()
    assert accepts_fp8_kv("economize") and not accepts_fp8_kv("sdpa")
    assert accepts_packed_kv("economize", "kivi") and accepts_packed_kv("economize", "quest")
    assert accepts_packed_kv("economize", "gathered") and not accepts_packed_kv("eager", "kivi")
    FusedFP8KVConfig().validate("economize")
    FusedKIVIConfig().validate("economize")
    QuestConfig().validate("economize")
    with pytest.raises(IncompatibleTechniquesError, match="economize"):
        FusedKIVIConfig().validate("sdpa")
    with pytest.raises(IncompatibleTechniquesError, match="fp8"):
        FusedFP8KVConfig().validate("eager")


def test_fp8_technique_makes_a_paged_cache() -> None:
    cache = technique_for(FP8KVConfig()).make_cache(pages=3, kv_heads=2, head_dim=64, device="cpu")
    assert isinstance(cache, PagedKVCache) and cache.dtype == torch.float8_e4m3fn
    assert cache.keys.shape == (3, 2, 4, 16, 16) and cache.values.shape == (3, 2, 64, 16)
    with pytest.raises(ConfigError, match="per-head"):
        technique_for(FP8KVConfig(scale="token")).make_cache(pages=3, kv_heads=2, head_dim=64, device="cpu")
    with pytest.raises(ConfigError, match="scales"):
        technique_for(FP8KVConfig(scale="head")).make_cache(pages=3, kv_heads=2, head_dim=64, device="cpu")


def test_paged_handle_formats_and_refusals() -> None:
    """The paged handle names its format; a bare handle (no dense stand-ins to materialize) cannot fall back, so a
    call the kernels do not take (here: CPU tensors) is refused, as is a handle over something that is not a paged
    cache."""
    cache = PagedKVCache.empty(2, 1, 64, torch.bfloat16, "cpu")
    table = torch.zeros(1, 2, dtype=torch.int32)
    kv = PagedKV(cache, table, torch.tensor([5], dtype=torch.int32), 5)
    assert kv.format == "bf16"
    q = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16)
    forward = ATTENTION_KERNELS["economize"].forward
    assert forward is economize_attention_forward
    with pytest.raises(ConfigError, match="cannot fall back"):
        forward(None, q, kv, None, None)
    with pytest.raises(ConfigError, match="no economize kernel"):
        PagedKV(object(), table, torch.tensor([5], dtype=torch.int32), 5)
    fp8 = PagedKV(PagedKVCache.empty(2, 1, 64, torch.float8_e5m2, "cpu"), table, kv.seq_lens, 5)
    assert fp8.format == "fp8"


def test_cached_workspace_clears_counters_a_previous_call_may_have_dirtied() -> None:
    """A call leaves its counters zero and may write partials after them; a later call with more counters gets the
    bytes in between cleared (a stale partial byte read as a counter miscounts a row's pieces)."""
    from economize_amd.paged import CachedWorkspace, counter_bytes

    assert counter_bytes(1, 1) == 256 and counter_bytes(70, 2) == 768 and counter_bytes(64, 1) == 256
    ws = CachedWorkspace()
    buf = ws.take(4096, counter_bytes(8, 8), "cpu")  # 256 counter bytes
    assert ws.zero_prefix == 256 and int(buf.sum()) == 0
    buf[256:].fill_(7)  # the call's partials
    again = ws.take(4096, counter_bytes(8, 8), "cpu")
    assert again is buf and int(buf[256:300].sum()) > 0  # same counters: nothing to clear
    ws.take(4096, counter_bytes(70, 2), "cpu")  # 768 counter bytes
    assert int(buf[:768].sum()) == 0 and int(buf[768:].min()) == 7
    grown = ws.take(8192, counter_bytes(70, 2), "cpu")
    assert grown.numel() == 8192 and int(grown.sum()) == 0


def test_a_kivi_pass_longer_than_the_headroom_is_refused() -> None:
    """The reference's test_a_pass_longer_than_the_headroom_is_refused (tests/techniques/test_kv_kivi_packed.py:
    151-155): a commit of more tokens than the ring holds beyond the residual would overwrite ring entries not yet
    quantized, so it raises before anything runs."""
    from economize_amd.kivi import PagedKIVICache, kivi_commit

    cache = PagedKIVICache.empty(4, 1, 1, 64, 2, "cpu", residual=32, headroom=32)
    with pytest.raises(ConfigError, match="headroom"):
        kivi_commit(cache, torch.zeros(1, 4, dtype=torch.int32), torch.zeros(1, dtype=torch.int32), 33)

