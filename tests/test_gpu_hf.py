"""End to end on the GPU: a small Qwen2 (bf16, head dim 64, GQA 2) decodes greedily with
``attn_implementation="economize"`` and its K/V in the techniques' paged caches (``economize_amd.hf.apply``), as the
reference compares its fused techniques with the plain ones on ``sdpa`` (tests/techniques/test_kv_fp8_fused.py:100-120,
test_kv_kivi_fused.py:124-138). Three checks:

* what the caches hold: fp8's greedy tokens equal those of ``sdpa`` over a dense cache of the fp8 round trip of every
  K/V (torch's own casts, the reference's fp8_encode / fp8_decode with no scale); KIVI's first layer, whose K/V
  depend on the token embeddings alone, holds bit for bit what the oracle's fake quantization (rounded to bf16) gives
  on the same schedule (keys below (c // R) * R, values below c - R quantized at every pass boundary);
* what the kernels compute over them: at every decoding step, a mirror of the model whose layers read the economize
  caches' dense view (the gather kernels) and attend with ``sdpa`` (Quest: over the oracle's select_pages and the
  tail, attention/quest.py) gives the logits of the economize run within a stated tolerance;
* that the paths run: the prompt (70 tokens, longer than the kernels take) on the fallback, every decoding step of a
  covered layer on the paged kernels (Quest on fp16 / fp32 models: the dense kernel's page list), as the usage log
  shows.

The dense runs of KIVI and Quest are not compared token for token: the later layers' K/V carry the rounding of the
earlier layers' attention (a bf16 MFMA kernel against ``sdpa``), and a 2-bit code or a page choice that this rounding
flips moves a logit by far more than rounding, after which greedy decoding may part. The checks above hold each part
to its own bar instead.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers.cache_utils import Cache, CacheLayerMixin, DynamicLayer

from oracle import kivi as okivi
from oracle import quest as oquest
from oracle.numerics import round_bf16

pytestmark = pytest.mark.gpu

PROMPT, STEPS = 70, 40


def tiny_model(attn: str, dtype: torch.dtype = torch.bfloat16, head_dim: int = 64):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    config = Qwen2Config(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=4,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=head_dim, max_position_embeddings=512,
                         tie_word_embeddings=True, initializer_range=0.2, attn_implementation=attn)
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(config).to(dtype).cuda().eval()
    model.requires_grad_(False)
    return model


def prompt() -> torch.Tensor:
    return torch.randint(0, 128, (1, PROMPT), generator=torch.Generator().manual_seed(1)).cuda()


@torch.no_grad()
def greedy(model, cache, ids: torch.Tensor, steps: int) -> list[int]:
    out = model(input_ids=ids, past_key_values=cache, use_cache=True)
    tokens = []
    for _ in range(steps):
        token = out.logits[:, -1].argmax(-1, keepdim=True)
        tokens.append(int(token))
        out = model(input_ids=token, past_key_values=cache, use_cache=True)
    return tokens


# ---- dense caches holding what the formats give -----------------------------------------------------------------


class FP8RoundTrip(DynamicLayer):
    def update(self, key_states, value_states, *args, **kwargs):
        def trip(x):
            return x.float().clamp(-448.0, 448.0).to(torch.float8_e4m3fn).to(x.dtype)

        return super().update(trip(key_states), trip(value_states))


class KIVIFakeQuant(DynamicLayer):
    """Dense K/V whose committed tokens are fake-quantized on KIVI's schedule at every pass boundary."""

    def __init__(self, bits: int, residual: int) -> None:
        super().__init__()
        self.bits, self.residual = bits, residual
        self.committed = self.kq = self.vq = 0

    def update(self, key_states, value_states, *args, **kwargs):
        length = self.get_seq_length()
        if length > self.committed:
            r = self.residual
            kq, vq = max(self.kq, (length // r) * r), max(self.vq, length - r)
            if kq > self.kq:
                block = self.keys[:, :, self.kq:kq].float().cpu().numpy()
                b, h, t, d = block.shape
                fq = okivi.fake_quantize(block.reshape(b, h, t // 32, 32, d), self.bits, axis=3).reshape(block.shape)
                self.keys[:, :, self.kq:kq] = torch.from_numpy(round_bf16(fq)).to(self.keys)
            if vq > self.vq:
                block = self.values[:, :, self.vq:vq].float().cpu().numpy()
                b, h, t, d = block.shape
                fq = okivi.fake_quantize(block.reshape(b, h, t, d // 32, 32), self.bits, axis=4).reshape(block.shape)
                self.values[:, :, self.vq:vq] = torch.from_numpy(round_bf16(fq)).to(self.values)
            self.kq, self.vq, self.committed = kq, vq, length
        return super().update(key_states, value_states)


def quest_oracle_forward(module, query, key, value, attention_mask, dropout=0.0, scaling=None, is_causal=None,
                         **kwargs):
    """``sdpa``, or, for a key carrying (done, page, selected pages), the oracle's attention over those pages and the
    tail (quest_reference)."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    info = getattr(key, "_quest", None)
    if info is None:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      is_causal=is_causal, **kwargs)
    done, page, index = info
    q = query.float().cpu().numpy()
    k = key.float().cpu().numpy()
    v = value.float().cpu().numpy()
    dones = np.full(q.shape[0], done, np.int32)
    mask = None if attention_mask is None else attention_mask[..., : k.shape[2]].cpu().numpy()
    out = oquest.quest_reference(q, k, v, mask, scaling, index, dones, page)
    return torch.from_numpy(out).to(query.device, query.dtype), None


class Mirror(CacheLayerMixin):
    """A layer that holds nothing: after the economize model's pass has written its tokens, it hands the mirror model
    the dense view of the economize layer (``materialized_kv``; a dense layer's own K/V), with the pages that pass
    selected on the key when it attended over Quest's pages."""

    is_sliding = False

    def __init__(self, source) -> None:
        super().__init__()
        self.source, self.tokens, self.selected = source, 0, None
        self.is_initialized = True

    def lazy_initialization(self, key_states, value_states) -> None:
        pass

    def get_seq_length(self) -> int:
        return self.source.get_seq_length() - self.tokens

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_max_length(self) -> int:
        return -1

    def update(self, key_states, value_states, *args, **kwargs):
        from economize_amd.hf import DenseFP8Layer, DenseQuestLayer, PackedKIVILayer, SimulatedKIVILayer
        from economize_amd.packed import materialized_kv

        if isinstance(self.source, DynamicLayer):
            return self.source.keys, self.source.values
        if isinstance(self.source, (DenseQuestLayer, SimulatedKIVILayer)):
            keys, values = (b[:, :, : self.source.length] for b in self.source.buffers)
        elif isinstance(self.source, PackedKIVILayer):  # the codes dequantized, the rings above them
            keys, values = self.source._dense(self.source.length)
        elif isinstance(self.source, DenseFP8Layer):  # the codes decoded to the model's dtype
            keys, values = (self.source._decoded(c[:, :, : self.source.length], i)
                            for i, c in enumerate(self.source.codes))
        else:
            keys, values = materialized_kv(*self.source.transform_read(key_states, value_states))
            if getattr(self.source, "quest", None) is not None:
                self.source._read(self.source.layer_idx)  # the mirror reads the same pages (through the oracle)
        keys = keys.view(keys.shape)
        if self.selected is not None:
            keys._quest = self.selected
        return keys, values


def mirrored_decode(configs, attn: str, dtype: torch.dtype = torch.bfloat16, head_dim: int = 64
                    ) -> tuple[list[float], list[float], set, int]:
    """Greedy decoding on the economize caches; after every pass the mirror model runs the same tokens over the
    caches' dense view. Every Quest selection of the economize pass is checked against the oracle's select_pages on
    the same query and bounds, and the mirror attends over the pages it chose. Returns each decoding step's largest
    logit difference, the mirror's top-2 gap at that step, the kernel paths the economize passes took and the number
    of selections checked."""
    from economize_amd.attention import kernel_usage
    from economize_amd.hf import DenseQuestLayer, apply
    from economize_amd.quest import QuestPages

    model = tiny_model("sdpa", dtype, head_dim)
    em = apply(model, *configs)
    cache = em.make_cache(PROMPT + STEPS + 1)
    mirror_model = tiny_model(attn, dtype, head_dim)
    layers = [Mirror(layer) for layer in cache.layers]
    mirror = Cache(layers=layers)
    selections = []
    select = QuestPages.select

    def recording_select(pages, query):
        index = select(pages, query)
        selections.append((pages, query.float().cpu().numpy(), index.cpu().numpy()))
        return index

    kernel_usage(reset=True)
    deltas, gaps, checked = [], [], 0
    ids = prompt()
    QuestPages.select = recording_select
    try:
        with torch.no_grad():
            for step in range(STEPS + 1):
                selections.clear()
                out = model(input_ids=ids, past_key_values=cache, use_cache=True)
                quest_layers = [m for m in layers if isinstance(m.source, DenseQuestLayer) or
                                getattr(m.source, "quest", None) is not None]
                for layer in layers:
                    layer.tokens, layer.selected = ids.shape[1], None
                if selections:
                    assert len(selections) == len(quest_layers)
                    for layer, (pages, query, index) in zip(quest_layers, selections):
                        want = oquest.select_pages(query, pages.kmin.float().cpu().numpy(),
                                                   pages.kmax.float().cpu().numpy(), pages.done.cpu().numpy(),
                                                   pages.max_done, pages.pages)
                        assert np.array_equal(index, want), step
                        layer.selected = (pages.max_done, pages.page, index)
                        checked += 1
                ref = mirror_model(input_ids=ids, past_key_values=mirror, use_cache=True)
                if step:
                    got, want = out.logits[0, -1].float(), ref.logits[0, -1].float()
                    deltas.append(float((got - want).abs().max()))
                    top = want.topk(2).values
                    gaps.append(float(top[0] - top[1]))
                ids = out.logits[:, -1].argmax(-1, keepdim=True)
    finally:
        QuestPages.select = select
    paths = {(row["path"], row["queries"]) for row in kernel_usage(reset=True)}
    return deltas, gaps, paths, checked


def dense_run(layers, attn: str) -> list[int]:
    model = tiny_model(attn)
    return greedy(model, Cache(layers=layers), prompt(), STEPS)


def economize_run(*configs) -> tuple[list[int], set]:
    from economize_amd.attention import kernel_usage
    from economize_amd.hf import apply

    model = tiny_model("sdpa")
    em = apply(model, *configs)
    kernel_usage(reset=True)
    tokens = greedy(model, em.make_cache(PROMPT + STEPS + 1), prompt(), STEPS)
    paths = {(row["path"], row["queries"]) for row in kernel_usage(reset=True)}
    return tokens, paths


def test_fp8_decodes_like_the_fp8_round_trip_on_sdpa() -> None:
    from economize_amd.techniques import FusedFP8KVConfig

    got, paths = economize_run(FusedFP8KVConfig())
    assert ("kernel_fp8", 1) in paths and ("sdpa", PROMPT) in paths
    assert got == dense_run([FP8RoundTrip() for _ in range(4)], "sdpa")


@pytest.mark.parametrize("bits", [2, 4])
def test_kivi_first_layer_holds_the_fake_quantization(bits: int) -> None:
    """Every decoding step: the first layer's dense view (quantized keys and values dequantized, the rest from the
    ring) equals the fake-quantized dense cache of a model fed the same tokens, bit for bit."""
    from economize_amd.hf import apply
    from economize_amd.kivi import kivi_gather
    from economize_amd.techniques import FusedKIVIConfig

    model = tiny_model("sdpa")
    em = apply(model, FusedKIVIConfig(bits=bits, residual_length=32, headroom=64))
    cache = em.make_cache(PROMPT + STEPS + 1)
    sim_model = tiny_model("sdpa")
    sim = Cache(layers=[KIVIFakeQuant(bits, 32) for _ in range(4)])
    ids = prompt()
    quantized = set()
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)
        sim_model(input_ids=ids, past_key_values=sim, use_cache=True)
        for step in range(STEPS):
            token = out.logits[:, -1].argmax(-1, keepdim=True)
            out = model(input_ids=token, past_key_values=cache, use_cache=True)
            sim_model(input_ids=token, past_key_values=sim, use_cache=True)
            layer, ref = cache.layers[0], sim.layers[0]
            assert (layer.kq, layer.vq) == (ref.kq, ref.vq), step
            keys, values = kivi_gather(layer.cache, layer.table, layer.length)
            assert torch.equal(keys, ref.keys) and torch.equal(values, ref.values), step
            quantized.add(layer.kq)
    assert quantized == {64, 96}  # the prompt's keys, then a group committed from the ring


#: Largest logit difference between the kernels and sdpa over the same cache: the rounding of bf16 activations and
#: of a bf16 MFMA kernel against sdpa, through four layers (observed: at most 0.23 over 40 steps of each technique).
LOGIT_TOL = 0.5


@pytest.mark.parametrize("technique", ["fp8", "kivi2", "kivi4", "quest", "quest_fp16", "quest_fp32", "fp8_d512",
                                       "kivi2_d512", "quest_d512", "kivi8_fp16", "kivi4_g16", "packed8",
                                       "packed4_g16_fp16", "packed2_d512", "fp8_fp16"])
def test_decoding_logits_match_sdpa_over_the_cache(technique: str) -> None:
    """Heads of 512 channels (``_d512``) run on the dense kernel's two value slices: dense fp8 buffers, KIVI codes in
    the reference's dense layout and Quest over dense buffers. ``kivi8_fp16`` (8-bit codes on an fp16 model) and
    ``kivi4_g16`` (groups of 16) are configurations the paged KIVI cache does not hold: the codes beside dense
    buffers, read by the kernel. ``packed*``: ``KIVIConfig``'s packed record and rings for such configurations, no
    dense buffer."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    from economize_amd.techniques import FusedFP8KVConfig, FusedKIVIConfig, KIVIConfig, QuestConfig

    attn, path, dtype = "sdpa", "kernel_fp8", torch.bfloat16
    head_dim = 512 if technique.endswith("_d512") else 64
    technique = technique.removesuffix("_d512")
    if technique in ("quest_fp16", "kivi8_fp16", "packed4_g16_fp16", "fp8_fp16"):
        dtype = torch.float16  # (fp8_fp16: an fp16 model over the paged fp8 cache, fp16 queries on the paged kernel)
    elif technique == "quest_fp32":
        dtype = torch.float32
    if technique in ("fp8", "fp8_fp16"):
        configs = (FusedFP8KVConfig(),)
    elif technique.startswith("kivi"):
        group = 16 if technique.endswith("_g16") else 32
        configs = (FusedKIVIConfig(bits=int(technique[4]), group_size=group, residual_length=32, headroom=64),)
        path = "kernel_kivi"
    elif technique.startswith("packed"):
        group = 16 if "_g16" in technique else 32
        configs = (KIVIConfig(bits=int(technique[6]), group_size=group, residual_length=32, headroom=64),)
        path = "kernel_kivi"
    else:
        configs = (QuestConfig(page_size=16, token_budget=64, dense_layers=1),)
        attn, path = "quest_oracle", "kernel_quest"
        AttentionInterface.register("quest_oracle", quest_oracle_forward)
        AttentionMaskInterface.register("quest_oracle", AttentionMaskInterface._global_mapping["sdpa"])
    if head_dim == 512 and technique == "fp8":
        path = "kernel"  # dense fp8 buffers
    deltas, gaps, paths, checked = mirrored_decode(configs, attn, dtype, head_dim)
    print(technique, head_dim, "max delta", max(deltas), "deltas", [round(d, 4) for d in deltas])
    assert (path, 1) in paths and ("sdpa", PROMPT) in paths
    if technique.startswith("quest"):  # (fp16 / fp32 models keep dense buffers: the dense kernel's page list)
        assert ("kernel", 1) in paths  # the dense first layer: the dense kernel
        # every decoding step commits at least 70 tokens, 4 full 16-token pages > 3 read: 3 covered layers select
        assert checked == 3 * STEPS
    assert max(deltas) <= LOGIT_TOL


def test_generate_runs_on_the_cache() -> None:
    """transformers' generate over the cache gives the greedy loop's tokens."""
    from economize_amd.hf import apply
    from economize_amd.techniques import FusedFP8KVConfig

    model = tiny_model("sdpa")
    em = apply(model, FusedFP8KVConfig())
    ids = prompt()
    out = em.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=12, pad_token_id=0)
    assert out[0, PROMPT:].tolist() == greedy(model, em.make_cache(PROMPT + 13), ids, 12)


# ---- the reference's golden model (float32, head dim 16): dense fp8 buffers on the dense kernel ------------------


class FP8Sim(DynamicLayer):
    """CPU K/V through the oracle's fp8 round trip with the reference's scale modes (fp8.py:81-97): ``"token"``, or
    a static scale (``"tensor"``)."""

    def __init__(self, mode: str, scales: tuple[float, float] | None = None) -> None:
        super().__init__()
        self.mode, self.scales = mode, scales

    def update(self, key_states, value_states, *args, **kwargs):
        from oracle import fp8 as ofp8

        def trip(x: torch.Tensor, i: int) -> torch.Tensor:
            x = x.numpy()
            scale = ofp8.token_scale(x, "e4m3") if self.mode == "token" else np.float32(self.scales[i])
            raw = ofp8.fp8_encode(x, "e4m3", scale)
            return torch.from_numpy(ofp8.fp8_decode(raw, "e4m3", scale, out="f32"))

        return super().update(trip(key_states, 0), trip(value_states, 1))


@torch.no_grad()
def golden_greedy(model, cache, device: str) -> list[int]:
    import test_golden_reference as golden

    out = model(input_ids=golden.prompt()[None].to(device), past_key_values=cache, use_cache=True)
    tokens = []
    for _ in range(golden.NEW_TOKENS):
        token = out.logits[:, -1].argmax(-1, keepdim=True)
        tokens.append(int(token))
        out = model(input_ids=token, past_key_values=cache, use_cache=True)
    return tokens


def test_the_hip_path_decodes_the_reference_fp8_golden_tokens() -> None:
    """The reference's own golden tokens of ``FP8KVConfig()`` (tests/golden/catalog.py:168-170, computed on the CPU)
    from its golden model on the GPU: ``kv_fp8_fused``'s dense fp8 buffers written by ``eco_fp8_encode`` and read as
    fp8 by the dense decode kernel at every decoding step (fp32 queries as exact bf16 hi + lo MFMA operands)."""
    import test_golden_reference as golden

    from economize_amd.attention import kernel_usage
    from economize_amd.hf import DenseFP8Layer, apply
    from economize_amd.techniques import FusedFP8KVConfig

    model = golden.golden_model().cuda()
    em = apply(model, FusedFP8KVConfig())
    cache = em.make_cache(golden.PROMPT + golden.NEW_TOKENS + 1)
    assert all(isinstance(layer, DenseFP8Layer) and layer.fused for layer in cache.layers)
    kernel_usage(reset=True)
    assert golden_greedy(model, cache, "cuda") == golden.GOLDEN["kv_fp8_tokens"].tolist()
    assert {(r["path"], r["queries"]) for r in kernel_usage(reset=True)} >= {("kernel", 1)}


def test_per_token_fp8_scales_decode_like_the_oracle() -> None:
    """``FP8KVConfig(scale="token")`` on the golden model: codes and per-token scales by ``eco_fp8_encode``, decoded
    to fp32 for the dense kernel, give the tokens of the CPU model over the oracle's per-token round trip."""
    import test_golden_reference as golden

    from economize_amd.hf import apply
    from economize_amd.techniques import FP8KVConfig

    want = golden_greedy(golden.golden_model(), Cache(layers=[FP8Sim("token") for _ in range(6)]), "cpu")
    model = golden.golden_model().cuda()
    em = apply(model, FP8KVConfig(scale="token"))
    assert golden_greedy(model, em.make_cache(64), "cuda") == want


def test_tensor_fp8_scales_are_calibrated_and_decode_like_the_oracle() -> None:
    """``FP8KVConfig(scale="tensor")`` calibrated on token batches at ``apply`` (calibrate_kv_absmax +
    static_scales, fp8.py:100-133): the per-layer scales are the CPU model's within fp32 noise, and decoding gives the
    tokens of the CPU model over the oracle's round trip with the same scales."""
    import test_golden_reference as golden
    from transformers import DynamicCache

    from economize_amd.hf import apply
    from economize_amd.techniques import FP8KVConfig

    batches = [golden._tokens(3, 8, 32)]
    cpu_model = golden.golden_model()
    absmax = torch.zeros(2, 6)

    class Recording(DynamicCache):
        def update(self, key_states, value_states, layer_idx, *args, **kwargs):
            absmax[0, layer_idx] = max(absmax[0, layer_idx], key_states.abs().amax())
            absmax[1, layer_idx] = max(absmax[1, layer_idx], value_states.abs().amax())
            return super().update(key_states, value_states, layer_idx, *args, **kwargs)

    with torch.no_grad():
        cpu_model(input_ids=batches[0], past_key_values=Recording(config=cpu_model.config), use_cache=True)
    model = golden.golden_model().cuda()
    em = apply(model, FP8KVConfig(scale="tensor"), calibration=batches)
    scales = torch.stack([torch.stack([em.scales[i][j][0] for i in range(6)]) for j in range(2)])
    torch.testing.assert_close(scales, absmax / 448.0, rtol=1e-5, atol=0)
    assert all((em.scales[i][j] == em.scales[i][j][0]).all() for i in range(6) for j in range(2))
    layers = [FP8Sim("tensor", (float(em.scales[i][0][0]), float(em.scales[i][1][0]))) for i in range(6)]
    want = golden_greedy(golden.golden_model(), Cache(layers=layers), "cpu")
    assert golden_greedy(model, em.make_cache(64), "cuda") == want


@pytest.mark.parametrize("storage", [None, "simulated"])
def test_the_hip_path_decodes_the_reference_kivi_golden_tokens(storage) -> None:
    """The reference's own golden tokens of ``KIVIConfig(bits=2, group_size=4, residual_length=8)``
    (tests/golden/catalog.py:163-165) from its golden model on the GPU. Groups of 4 are not the paged cache's: with
    the default storage the layers keep the reference's packed record and rings (:class:`PackedKIVILayer`, no dense
    buffer; every decoding step's kernel reads the codes and the rings), with ``storage="simulated"`` dense buffers
    quantized in place by ``eco_kivi_fake_quantize`` at every pass boundary, read by the dense kernel."""
    import test_golden_reference as golden

    from economize_amd.attention import kernel_usage
    from economize_amd.hf import PackedKIVILayer, SimulatedKIVILayer, apply
    from economize_amd.techniques import KIVIConfig

    model = golden.golden_model().cuda()
    em = apply(model, KIVIConfig(bits=2, group_size=4, residual_length=8, storage=storage))
    cache = em.make_cache(golden.PROMPT + golden.NEW_TOKENS + 1)
    layer_class, path = (SimulatedKIVILayer, "kernel") if storage else (PackedKIVILayer, "kernel_kivi")
    assert all(type(layer) is layer_class for layer in cache.layers)
    kernel_usage(reset=True)
    assert golden_greedy(model, cache, "cuda") == golden.GOLDEN["kv_kivi_2bit_tokens"].tolist()
    assert {(r["path"], r["queries"]) for r in kernel_usage(reset=True)} >= {(path, 1)}
    assert (cache.layers[0].kq, cache.layers[0].vq) == (32, 31)  # 39 committed tokens before the last pass


def test_the_reference_kivi_golden_tokens_through_the_codes() -> None:
    """The same golden case as ``FusedKIVIConfig``: the layers keep the reference's packed codes beside the dense
    buffers (:class:`FusedKIVIDenseLayer`) and every decoding step's kernel reads the quantized prefix through the
    codes (``eco_kivi_packed_decode``); the tokens are the reference's ``kv_kivi_2bit`` ones."""
    import test_golden_reference as golden

    from economize_amd.attention import kernel_usage
    from economize_amd.hf import FusedKIVIDenseLayer, apply
    from economize_amd.techniques import FusedKIVIConfig

    model = golden.golden_model().cuda()
    em = apply(model, FusedKIVIConfig(bits=2, group_size=4, residual_length=8))
    cache = em.make_cache(golden.PROMPT + golden.NEW_TOKENS + 1)
    assert all(isinstance(layer, FusedKIVIDenseLayer) for layer in cache.layers)
    kernel_usage(reset=True)
    assert golden_greedy(model, cache, "cuda") == golden.GOLDEN["kv_kivi_2bit_tokens"].tolist()
    assert {(r["path"], r["queries"]) for r in kernel_usage(reset=True)} >= {("kernel_kivi", 1)}
    layer = cache.layers[0]
    assert (layer.kq, layer.vq) == (32, 31) and layer.packable
    assert layer.store.keys_quantized.tolist() == [32] and layer.store.values_quantized.tolist() == [31]


def test_the_hip_path_decodes_the_reference_quest_golden_tokens() -> None:
    """The reference's own golden tokens of ``QuestConfig(page_size=16, token_budget=32, dense_layers=0)``
    (tests/golden/catalog.py:195-207) from its golden model on the GPU: float32 at head dim 16, so the layers keep
    dense buffers (:class:`DenseQuestLayer`) with their bounds computed by ``eco_quest_dense_bounds``, and every
    decoding step past two committed pages selects its page by ``eco_quest_select`` and attends over it and the tail
    by ``eco_quest_decode``."""
    import test_golden_reference as golden

    from economize_amd.attention import kernel_usage
    from economize_amd.hf import DenseQuestLayer, apply
    from economize_amd.techniques import QuestConfig

    model = golden.golden_model().cuda()
    em = apply(model, QuestConfig(page_size=16, token_budget=32, dense_layers=0))
    cache = em.make_cache(golden.PROMPT + golden.NEW_TOKENS + 1)
    assert all(isinstance(layer, DenseQuestLayer) for layer in cache.layers)
    kernel_usage(reset=True)
    assert golden_greedy(model, cache, "cuda") == golden.GOLDEN["kv_quest_tokens"].tolist()
    usage = kernel_usage(reset=True)
    quest_calls = sum(row["calls"] for row in usage if row["path"] == "kernel_quest")
    # steps at 32 .. 39 committed tokens: two committed pages, more than the one page read, in each of 6 layers
    assert quest_calls == 6 * (golden.PROMPT + golden.NEW_TOKENS - 32)
    assert {(row["path"], row["queries"]) for row in usage} >= {("kernel", 1), ("kernel_quest", 1)}


def _quest_call(layer: int, dtype: torch.dtype, paged: bool):
    """A decoding call of a Quest layer: the module, a query, and K/V carrying the layer's pages (a paged bf16 cache's
    handle, or QuestPages on dense buffers), with the oracle's inputs."""
    from economize_amd.attention import PagedKV
    from economize_amd.packed import attach_packed, stand_in
    from economize_amd.paged import PAGE, PagedKVCache, paged_append
    from economize_amd.quest import QuestPages, page_bounds, paged_page_bounds

    model = tiny_model("economize", dtype)
    module = model.model.layers[layer].self_attn
    gen = torch.Generator().manual_seed(layer)
    batch, hq, hkv, slots, d, page, pages = 2, 4, 2, 300, 64, 16, 4
    q = torch.randn(batch, hq, 1, d, generator=gen).to(dtype).cuda()
    k = torch.randn(batch, hkv, slots, d, generator=gen).to(dtype).cuda()
    v = torch.randn(batch, hkv, slots, d, generator=gen).to(dtype).cuda()
    done = slots // page
    done_t = torch.full((batch,), done, dtype=torch.int32, device="cuda")
    if not paged:
        kmin, kmax = page_bounds(k, 0, done, page)
        qp = QuestPages(kmin, kmax, done_t, done, done, page, pages)
        return module, q, attach_packed(k, qp), v, k, v, qp
    table = torch.arange(batch * -(-slots // PAGE), dtype=torch.int32, device="cuda").view(batch, -1)
    cache = PagedKVCache.empty(table.numel(), hkv, d, torch.bfloat16, "cuda")
    pos = torch.arange(slots, device="cuda")
    slot_ids = (table[:, pos // PAGE] * PAGE + pos % PAGE).to(torch.int32).reshape(-1)
    paged_append(cache, k.transpose(1, 2).reshape(-1, hkv, d), v.transpose(1, 2).reshape(-1, hkv, d), slot_ids)
    kmin, kmax = paged_page_bounds(cache, table, 0, done, page)
    qp = QuestPages(kmin, kmax, done_t, done, done, page, pages)
    lens = torch.full((batch,), slots, dtype=torch.int32, device="cuda")
    handle = PagedKV(cache, table, lens, slots, qp, dtype)
    stand = stand_in((batch, hkv, slots, d), dtype, q.device)
    return module, q, attach_packed(stand, handle), stand, k, v, qp


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("why", ["output_attentions", "float_mask"])
def test_a_quest_call_that_falls_back_reads_the_selected_pages_only(paged: bool, why: str) -> None:
    """A Quest call the kernels do not run (attention weights asked for: the model's eager function; an additive
    float mask: sdpa) hides the unselected pages in its mask before it attends, as the reference's fallback does
    (interface.py:216-222, QuestPages.restrict_mask): its output equals the oracle's quest_reference over the same
    pages, not the dense attention."""
    from economize_amd.attention import economize_attention_forward, kernel_usage
    from oracle.attention import reference_attention

    dtype = torch.bfloat16
    module, q, key, value, k, v, qp = _quest_call(1, dtype, paged)
    kwargs, mask = {}, None
    if why == "output_attentions":
        kwargs["output_attentions"] = True
    else:
        mask = torch.zeros(q.shape[0], 1, 1, k.shape[2], dtype=dtype, device="cuda")
    kernel_usage(reset=True)
    got, _ = economize_attention_forward(module, q, key, value, mask, scaling=0.125, **kwargs)
    assert [row["reason"] for row in kernel_usage(reset=True)] == [why]
    index = qp.select(q).cpu().numpy()
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    done = qp.done.cpu().numpy()
    want = oquest.quest_reference(f(q), f(k), f(v), None, 0.125, index, done, qp.page)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=2e-2, rtol=2e-2)
    dense = reference_attention(f(q), f(k), f(v), None, 0.125)
    assert np.abs(want - dense).max() > 0.05  # the restriction is visible at this tolerance


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quest_on_dense_buffers_runs_on_the_kernel(dtype) -> None:
    """The forward routes a dense key carrying QuestPages (an fp16 / fp32 model's Quest layer) to eco_quest_decode
    (path "kernel_quest"), within atol 2e-3 / rtol 1e-2 of the oracle."""
    from economize_amd.attention import economize_attention_forward, kernel_usage

    module, q, key, value, k, v, qp = _quest_call(2, dtype, paged=False)
    kernel_usage(reset=True)
    got, _ = economize_attention_forward(module, q, key, value, None, scaling=0.125)
    assert [(row["path"], row["reason"]) for row in kernel_usage(reset=True)] == [("kernel_quest", "")]
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    want = oquest.quest_reference(f(q), f(k), f(v), None, 0.125, qp.select(q).cpu().numpy(), qp.done.cpu().numpy(),
                                  qp.page)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quest_pages_no_attention_function_read_raise(dtype) -> None:
    """The reference's unread-pages check (techniques/quest/technique.py:174-182): a Quest layer whose attached pages
    no attention function read (the model switched to sdpa after apply) raises when it is written next, instead of
    decoding densely without a word; with the economize kernel the same steps run."""
    from economize_amd.errors import IncompatibleTechniquesError
    from economize_amd.hf import apply
    from economize_amd.techniques import QuestConfig

    model = tiny_model("sdpa", dtype)
    em = apply(model, QuestConfig(page_size=16, token_budget=32, dense_layers=0))
    ids = prompt()
    with torch.no_grad():
        greedy(model, em.make_cache(PROMPT + 4), ids, 3)  # the economize kernel reads every attachment
        model.set_attn_implementation("sdpa")
        cache = em.make_cache(PROMPT + 4)
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)  # the prompt: nothing attached
        token = out.logits[:, -1].argmax(-1, keepdim=True)
        model(input_ids=token, past_key_values=cache, use_cache=True)  # pages attached, read by nobody
        with pytest.raises(IncompatibleTechniquesError, match="no attention function read"):
            model(input_ids=token, past_key_values=cache, use_cache=True)
    model.set_attn_implementation("economize")


def test_a_captured_decode_step_of_a_quest_model_replays_like_eager() -> None:
    """Quest's metadata on the device inside the drop-in: a bf16 Qwen2 whose layers live in a static cache (paged,
    every length on the device; Quest's bounds refreshed by the append's own launch) is captured once, decoding step
    ``model(input_ids=token, position_ids=position, past_key_values=cache)`` with the token and position in device
    buffers, and replayed; a twin model stepping eagerly over a twin cache gives bit-identical logits at every step
    while the rows cross page boundaries (80, 96, 112 and 128 tokens) and Quest selects among more and more pages."""
    from economize_amd.attention import kernel_usage
    from economize_amd.hf import PagedLayer, apply
    from economize_amd.techniques import QuestConfig

    cap, steps = 200, 60

    def build():
        model = tiny_model("sdpa")
        em = apply(model, QuestConfig(page_size=16, token_budget=64, dense_layers=1))
        return model, em.make_cache(cap, static=True)

    (m0, c0), (m1, c1) = build(), build()
    assert all(isinstance(layer, PagedLayer) and layer.static for layer in c0.layers)
    assert [layer.quest is not None for layer in c0.layers] == [False, True, True, True]
    ids = prompt()
    pos = torch.arange(PROMPT, device="cuda")[None]
    kernel_usage(reset=True)
    with torch.no_grad():
        first = m0(input_ids=ids, position_ids=pos, past_key_values=c0, use_cache=True).logits
        assert torch.equal(first, m1(input_ids=ids, position_ids=pos, past_key_values=c1, use_cache=True).logits)
        token = torch.zeros(1, 1, dtype=torch.long, device="cuda")
        position = torch.zeros(1, 1, dtype=torch.long, device="cuda")
        token.copy_(first[:, -1].argmax(-1, keepdim=True))
        position.fill_(PROMPT)

        def step(model, cache):
            return model(input_ids=token, position_ids=position, past_key_values=cache, use_cache=True).logits

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up on a side stream: workspaces exist before the capture
            warm = step(m0, c0)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert torch.equal(warm, step(m1, c1))
        token.copy_(warm[:, -1].argmax(-1, keepdim=True))
        position += 1
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = step(m0, c0)
        # the capture recorded the step without running it: the first replay runs it
        for i in range(steps):
            graph.replay()
            torch.cuda.synchronize()
            eager = step(m1, c1)
            torch.cuda.synchronize()
            assert torch.equal(captured, eager), f"step {i}, position {int(position)}"
            token.copy_(eager[:, -1].argmax(-1, keepdim=True))
            position += 1
    assert int(position) == PROMPT + 1 + steps
    paths = {(row["path"], row["queries"]) for row in kernel_usage(reset=True)}
    assert ("kernel_quest", 1) in paths and ("kernel_bf16", 1) in paths
    for a, b in zip(c0.layers[1:], c1.layers[1:]):
        assert torch.equal(a.state.done, b.state.done) and torch.equal(a.state.kmin, b.state.kmin)
    assert int(c1.layers[1].state.done[0]) == (PROMPT + 1 + steps) // 16


def test_a_captured_decode_step_of_an_fp8_model_replays_like_eager() -> None:
    """The headline path inside the drop-in: a bf16 Qwen2 whose layers live in a static paged fp8 cache (every length
    on the device) is captured once, decoding step ``model(input_ids=token, position_ids=position,
    past_key_values=cache)`` with the token and position in device buffers, and replayed; a twin model stepping
    eagerly over a twin cache gives bit-identical logits at every step while the rows cross page boundaries."""
    from economize_amd.attention import kernel_usage
    from economize_amd.hf import PagedLayer, apply
    from economize_amd.techniques import FusedFP8KVConfig

    cap, steps = 200, 40

    def build():
        model = tiny_model("sdpa")
        em = apply(model, FusedFP8KVConfig())
        return model, em.make_cache(cap, static=True)

    (m0, c0), (m1, c1) = build(), build()
    assert all(isinstance(layer, PagedLayer) and layer.static for layer in c0.layers)
    ids = prompt()
    pos = torch.arange(PROMPT, device="cuda")[None]
    kernel_usage(reset=True)
    with torch.no_grad():
        first = m0(input_ids=ids, position_ids=pos, past_key_values=c0, use_cache=True).logits
        assert torch.equal(first, m1(input_ids=ids, position_ids=pos, past_key_values=c1, use_cache=True).logits)
        token = torch.zeros(1, 1, dtype=torch.long, device="cuda")
        position = torch.zeros(1, 1, dtype=torch.long, device="cuda")
        token.copy_(first[:, -1].argmax(-1, keepdim=True))
        position.fill_(PROMPT)

        def step(model, cache):
            return model(input_ids=token, position_ids=position, past_key_values=cache, use_cache=True).logits

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up on a side stream: workspaces exist before the capture
            warm = step(m0, c0)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert torch.equal(warm, step(m1, c1))
        token.copy_(warm[:, -1].argmax(-1, keepdim=True))
        position += 1
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = step(m0, c0)
        for i in range(steps):
            graph.replay()
            torch.cuda.synchronize()
            eager = step(m1, c1)
            torch.cuda.synchronize()
            assert torch.equal(captured, eager), f"step {i}, position {int(position)}"
            token.copy_(eager[:, -1].argmax(-1, keepdim=True))
            position += 1
    assert int(position) == PROMPT + 1 + steps
    paths = {(row["path"], row["queries"]) for row in kernel_usage(reset=True)}
    assert ("kernel_fp8", 1) in paths
