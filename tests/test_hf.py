"""The drop-in boundary on the CPU: the ``"economize"`` registration with transformers (attention/interface.py:
502-525), ``validate(adapter)`` refusing what the MI355X path cannot run before anything attaches, ``apply``'s
refusal of two techniques on one layer, and the forward's per-call fallback (a CPU call runs transformers' sdpa and
is logged with its reason, attention/interface.py:243-285)."""

from __future__ import annotations

import pytest
import torch

from economize_amd.errors import ConfigError, IncompatibleTechniquesError
from economize_amd.techniques import FP8KVConfig, FusedFP8KVConfig, FusedKIVIConfig, KIVIConfig, QuestConfig


def tiny_model(head_dim: int = 64, attn: str = "sdpa", layers: int = 4):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from economize_amd.attention import install

    install()  # a model built with attn="economize" needs the registration, whatever ran before in this process
    config = Qwen2Config(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=head_dim, max_position_embeddings=512,
                         tie_word_embeddings=True, initializer_range=0.2, attn_implementation=attn)
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(config).eval()
    model.requires_grad_(False)
    return model


def test_install_registers_the_forward_with_transformers() -> None:
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    from economize_amd.attention import economize_attention_forward, install

    assert "economize" in install()
    assert AttentionInterface._global_mapping["economize"] is economize_attention_forward
    assert AttentionMaskInterface._global_mapping["economize"] is AttentionMaskInterface._global_mapping["sdpa"]


def test_validate_refuses_what_the_path_cannot_run() -> None:
    model = tiny_model()
    model.config._attn_implementation = "economize"
    FusedFP8KVConfig().validate(model)
    FusedKIVIConfig().validate(model)
    QuestConfig().validate(model.config)
    for scale in ("none", "token", "tensor", "head"):
        FP8KVConfig(scale=scale).validate(tiny_model(head_dim=32))  # dense fp8 buffers take any head dim
    FusedFP8KVConfig().validate(tiny_model(head_dim=512, attn="economize"))  # fp8 buffers: up to 512
    with pytest.raises(ConfigError, match="up to 512"):
        FusedFP8KVConfig().validate(tiny_model(head_dim=640, attn="economize"))
    for config in (KIVIConfig(bits=8), KIVIConfig(group_size=64, residual_length=128), KIVIConfig(storage="simulated"),
                   KIVIConfig(bits=4, group_size=4, residual_length=8), KIVIConfig(bits=8, storage="packed"),
                   KIVIConfig(group_size=64, residual_length=128, storage="packed")):
        config.validate(model)  # the packed record and the simulated storage take what the paged cache cannot hold
    with pytest.raises(ConfigError, match="up to 256"):  # simulated buffers in the model's fp32
        FusedKIVIConfig().validate(tiny_model(head_dim=512, attn="economize"))
    FusedKIVIConfig().validate(tiny_model(head_dim=512, attn="economize").to(torch.bfloat16))
    with pytest.raises(ConfigError, match="up to 512"):
        FusedKIVIConfig().validate(tiny_model(head_dim=640, attn="economize").to(torch.bfloat16))
    with pytest.raises(IncompatibleTechniquesError, match="economize"):
        FusedFP8KVConfig().validate(tiny_model())  # the model runs sdpa


def test_apply_selects_the_kernel_and_refuses_conflicts() -> None:
    from economize_amd.hf import apply

    model = tiny_model()
    em = apply(model, FusedFP8KVConfig(layers=(1, 2)), QuestConfig(dense_layers=2))
    assert model.config._attn_implementation == "economize"
    assert [type(t.config).__name__ if t else None for t in map(em.technique_of, [1, 2, 3, 4])] == \
        ["FusedFP8KVConfig", "FusedFP8KVConfig", "QuestConfig", "QuestConfig"]
    with pytest.raises(IncompatibleTechniquesError, match="one KV technique per layer"):
        apply(tiny_model(), FusedFP8KVConfig(), FusedKIVIConfig())
    with pytest.raises(IncompatibleTechniquesError, match="twice"):
        apply(tiny_model(), FusedFP8KVConfig(layers=(1,)), FusedFP8KVConfig(layers=(2,)))
    with pytest.raises(ConfigError, match="calibrated at attach time"):
        apply(tiny_model(), FP8KVConfig(scale="tensor"))
    with pytest.raises(ConfigError, match="needs the paged fp8 cache"):
        apply(tiny_model(head_dim=32), FusedFP8KVConfig(scale="head"))


def test_fp8_layers_are_paged_where_the_paged_kernels_take_the_model() -> None:
    """bf16 models of head dim 64 / 128 / 256 keep fp8 layers in the paged cache (scale none, tensor or head); a
    per-token scale, another head dim or another dtype gets dense fp8 buffers (kv_fp8 decodes them for attention,
    kv_fp8_fused hands the fp8 views to the kernel)."""
    from economize_amd.hf import DenseFP8Layer, PagedLayer, apply

    def layer_types(model, config):
        cache = apply(model, config).make_cache(64)
        return [(type(layer).__name__, getattr(layer, "fused", None)) for layer in cache.layers[:1]]

    bf16 = tiny_model().to(torch.bfloat16)
    assert layer_types(bf16, FusedFP8KVConfig()) == [("PagedLayer", None)]
    assert layer_types(tiny_model().to(torch.bfloat16), FP8KVConfig(scale="token")) == [("DenseFP8Layer", False)]
    assert layer_types(tiny_model(head_dim=16).to(torch.bfloat16), FusedFP8KVConfig()) == [("DenseFP8Layer", True)]
    assert layer_types(tiny_model(), FusedFP8KVConfig()) == [("DenseFP8Layer", True)]  # float32
    assert PagedLayer and DenseFP8Layer


def test_a_cpu_call_falls_back_to_sdpa_and_is_logged() -> None:
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    from economize_amd.attention import economize_attention_forward, kernel_usage

    kernel_usage(reset=True)
    module = torch.nn.Module()
    module.layer_idx = 3
    module.is_causal = True
    module.num_key_value_groups = 2
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(1, 4, 1, 64, generator=gen)
    k = torch.randn(1, 2, 9, 64, generator=gen)
    v = torch.randn(1, 2, 9, 64, generator=gen)
    mask = torch.ones(1, 1, 1, 9, dtype=torch.bool)
    got, _ = economize_attention_forward(module, q, k, v, mask, scaling=0.125)
    want, _ = sdpa_attention_forward(module, q, k, v, mask, scaling=0.125)
    assert torch.equal(got, want)
    assert kernel_usage() == [{"layer": 3, "queries": 1, "path": "sdpa", "reason": "cpu", "calls": 1}]


def test_kivi_layers_are_paged_where_the_paged_cache_holds_them() -> None:
    """2- and 4-bit codes in groups of 32 on a bf16 model of head dim 64 / 128 live in the paged KIVI cache; 8-bit
    codes, other groups, head dims and dtypes keep the reference's packed record and rings (kv_quant/packed.py), or
    its codes beside dense buffers for FusedKIVIConfig (kv_kivi_fused/fused.py:104-250); storage='simulated' gets
    the simulated storage (kivi.py:62-66)."""
    from economize_amd.hf import apply

    def layer_type(model, config) -> str:
        return type(apply(model, config).make_cache(64).layers[0]).__name__

    bf16 = tiny_model().to(torch.bfloat16)
    assert layer_type(bf16, FusedKIVIConfig()) == "KIVILayer"
    assert layer_type(tiny_model().to(torch.bfloat16), KIVIConfig(bits=4)) == "KIVILayer"
    assert layer_type(tiny_model().to(torch.bfloat16), KIVIConfig(storage="simulated")) == "SimulatedKIVILayer"
    assert layer_type(tiny_model().to(torch.bfloat16), KIVIConfig(bits=8)) == "PackedKIVILayer"
    assert layer_type(tiny_model().to(torch.bfloat16), KIVIConfig(bits=8, storage="packed")) == "PackedKIVILayer"
    assert layer_type(tiny_model().to(torch.bfloat16), FusedKIVIConfig(group_size=16, residual_length=32)) == \
        "FusedKIVIDenseLayer"
    assert layer_type(tiny_model(head_dim=16).to(torch.bfloat16), KIVIConfig()) == "PackedKIVILayer"
    assert layer_type(tiny_model(), FusedKIVIConfig()) == "FusedKIVIDenseLayer"  # float32


def test_quest_layers_are_paged_where_the_paged_kernels_take_the_model() -> None:
    """Quest on a bf16 model of head dim 64 / 128 / 256 keeps its layers in the paged bf16 cache; fp16 / fp32 models
    and other head dims keep dense buffers of the model's dtype (the dense kernel's page list), and head dims the
    kernels do not take are refused before anything attaches."""
    from economize_amd.hf import DenseQuestLayer, PagedLayer, apply

    def layer_types(model) -> list[str]:
        cache = apply(model, QuestConfig(dense_layers=1)).make_cache(64)
        return [type(layer).__name__ for layer in cache.layers[:2]]

    assert layer_types(tiny_model().to(torch.bfloat16)) == ["DynamicLayer", "PagedLayer"]
    assert layer_types(tiny_model().to(torch.float16)) == ["DynamicLayer", "DenseQuestLayer"]
    assert layer_types(tiny_model()) == ["DynamicLayer", "DenseQuestLayer"]  # float32
    assert layer_types(tiny_model(head_dim=32).to(torch.bfloat16)) == ["DynamicLayer", "DenseQuestLayer"]
    assert layer_types(tiny_model(head_dim=512).to(torch.bfloat16)) == ["DynamicLayer", "DenseQuestLayer"]
    with pytest.raises(ConfigError, match="up to 256"):  # dense buffers in the model's fp32
        apply(tiny_model(head_dim=512), QuestConfig())
    with pytest.raises(ConfigError, match="multiples of 8"):
        apply(tiny_model(head_dim=36), QuestConfig())
    assert PagedLayer and DenseQuestLayer


def test_a_static_cache_holds_paged_layers_only() -> None:
    """``make_cache(static=True)``: every layer paged with device lengths (no technique: bf16 pages; fp8; Quest), and
    a refusal for what a static cache cannot hold (another dtype, KIVI, per-token fp8 scales)."""
    from economize_amd.hf import PagedLayer, apply

    bf16 = tiny_model().to(torch.bfloat16)
    cache = apply(bf16, FusedFP8KVConfig(layers=(1,)), QuestConfig(dense_layers=2)).make_cache(64, static=True)
    assert all(isinstance(layer, PagedLayer) and layer.static for layer in cache.layers)
    assert [layer.cache_dtype for layer in cache.layers] == [torch.float8_e4m3fn, None, None, None]
    assert [layer.quest is not None for layer in cache.layers] == [False, False, True, True]
    assert cache.layers[0].get_mask_sizes(1) == (64, 0)
    with pytest.raises(ConfigError, match="static cache takes a bf16 model"):
        apply(tiny_model(), QuestConfig()).make_cache(64, static=True)
    with pytest.raises(ConfigError, match="KIVIConfig"):
        apply(tiny_model().to(torch.bfloat16), KIVIConfig()).make_cache(64, static=True)
    with pytest.raises(ConfigError, match="FP8KVConfig"):
        apply(tiny_model().to(torch.bfloat16), FP8KVConfig(scale="token")).make_cache(64, static=True)
