"""The reference's own golden outputs, reproduced on the CPU with the oracle.

The reference pins its techniques end to end with golden tensors (tests/golden/cases.py, catalog.py; the data files
are copied into ``tests/golden/reference_golden.npz`` by ``tests/golden/make_fixtures.py``). The cases of this path
run a tiny float32 Qwen2 through greedy decoding with the technique's cache, so a token that moved would mean the
oracle's fp8 round trip, KIVI quantization and schedule or Quest selection differ from the reference's. Here the same
model decodes through transformers with cache layers and an attention function built on the oracle:

* ``dense``: the model recipe (cases.py:118-140: seeded float64 noise per parameter in name order) gives the
  reference's logits on the held-out sequence (the reference's tolerance, atol 1e-3 / rtol 1e-3);
* ``kv_fp8``: every K/V written through ``oracle.fp8`` encode and decode (fp8.py:81-92, scale ``"none"``);
* ``kv_kivi_2bit``: KIVI at 2 bits, groups of 4, residual 8: at every pass boundary keys below ``(c // 8) * 8`` and
  values below ``c - 8`` are fake-quantized with ``oracle.kivi`` (kivi.py:191-202, 230-275; the prompt once its pass
  has run);
* ``kv_quest``: decoding queries attend over ``oracle.quest``'s selected pages and the tail when more than the
  budget's pages are committed (quest/technique.py:194-227, attention/quest.py:73-108, 207-219).

Tokens must match exactly (the reference's rule for integer tensors, cases.py:104-107).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import kivi as okivi
from oracle import quest as oquest

transformers = pytest.importorskip("transformers")
from transformers.cache_utils import Cache, DynamicLayer  # noqa: E402

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "reference_golden.npz")
VOCAB, PROMPT, NEW_TOKENS = 128, 16, 24


def golden_model(attn: str = "sdpa") -> torch.nn.Module:
    """A 6-layer float32 Qwen2 (hidden 64, 4 query and 2 KV heads of 16 channels) whose parameters, in name order,
    are drawn from one float64 generator seeded 0: norms ``1 + 0.1 n``, biases ``0.02 n``, matrices ``0.2 n``."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    config = Qwen2Config(vocab_size=VOCAB, hidden_size=64, intermediate_size=128, num_hidden_layers=6,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                         tie_word_embeddings=True, initializer_range=0.2, attn_implementation=attn)
    model = Qwen2ForCausalLM(config).float().eval()
    model.requires_grad_(False)
    generator = torch.Generator().manual_seed(0)
    with torch.no_grad():
        for name, parameter in sorted(model.named_parameters()):
            noise = torch.randn(parameter.shape, generator=generator, dtype=torch.float64).float()
            if "norm" in name:
                parameter.copy_(1 + 0.1 * noise)
            elif name.endswith("bias"):
                parameter.copy_(0.02 * noise)
            else:
                parameter.copy_(0.2 * noise)
    return model


def _tokens(seed: int, *shape: int) -> torch.Tensor:
    return torch.randint(1, VOCAB, shape, generator=torch.Generator().manual_seed(seed))


def prompt() -> torch.Tensor:
    head = _tokens(1, PROMPT // 2)
    return torch.cat([head, head])


@torch.no_grad()
def greedy(model: torch.nn.Module, cache: Cache) -> list[int]:
    """The prompt in one pass, then one token per pass."""
    out = model(input_ids=prompt()[None], past_key_values=cache, use_cache=True)
    tokens = []
    for _ in range(NEW_TOKENS):
        token = out.logits[:, -1].argmax(-1, keepdim=True)
        tokens.append(int(token))
        out = model(input_ids=token, past_key_values=cache, use_cache=True)
    return tokens


class FP8Layer(DynamicLayer):
    """Dense K/V holding the oracle's e4m3 round trip of every entry."""

    def update(self, key_states, value_states, *args, **kwargs):
        def trip(x: torch.Tensor) -> torch.Tensor:
            raw = ofp8.fp8_encode(x.numpy(), "e4m3", None)
            return torch.from_numpy(ofp8.fp8_decode(raw, "e4m3", None, out="f32"))

        return super().update(trip(key_states), trip(value_states))


class KIVILayer(DynamicLayer):
    """Dense K/V whose committed entries are fake-quantized by the oracle on KIVI's schedule at every pass
    boundary; a prompt is quantized once its own pass has attended (kivi.py:204-214)."""

    def __init__(self, bits: int, group: int, residual: int) -> None:
        super().__init__()
        self.bits, self.group, self.residual = bits, group, residual
        self.kq = self.vq = 0

    def commit(self) -> None:
        k_to, v_to = okivi.schedule(self.get_seq_length(), self.residual)
        if k_to > self.kq:
            _, _, _, dense = okivi.quantize_keys(self.keys.numpy(), self.kq, k_to, self.bits, self.group)
            self.keys[:, :, self.kq:k_to] = torch.from_numpy(dense)
            self.kq = k_to
        if v_to > self.vq:
            _, _, _, dense = okivi.quantize_values(self.values.numpy(), self.vq, v_to, self.bits, self.group)
            self.values[:, :, self.vq:v_to] = torch.from_numpy(dense)
            self.vq = v_to

    def update(self, key_states, value_states, *args, **kwargs):
        if self.is_initialized:
            self.commit()  # the previous pass ended: everything before this pass is committed
        keys, values = super().update(key_states, value_states)
        return keys.clone(), values.clone()  # this pass attends before a later commit rewrites the buffers


class QuestLayer(DynamicLayer):
    """Dense K/V; a decoding query's key carries ``(done, page, pages)`` when more than ``pages`` pages are
    committed (quest/technique.py:194-227)."""

    def __init__(self, page: int, pages: int) -> None:
        super().__init__()
        self.page, self.pages = page, pages

    def update(self, key_states, value_states, *args, **kwargs):
        done = self.get_seq_length() // self.page
        keys, values = super().update(key_states, value_states)
        if key_states.shape[2] == 1 and done > self.pages:
            keys = keys.view(keys.shape)
            keys._quest = (done, self.page, self.pages)
        return keys, values


def quest_forward(module, query, key, value, attention_mask, dropout=0.0, scaling=None, is_causal=None, **kwargs):
    """``sdpa``, or the oracle's selection and restricted attention for a key carrying Quest's parameters."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    info = getattr(key, "_quest", None)
    if info is None:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      is_causal=is_causal, **kwargs)
    done, page, pages = info
    q, k, v = (t.float().numpy() for t in (query, key, value))
    dones = np.full(q.shape[0], done, np.int32)
    lo, hi = oquest.page_bounds(k, 0, done, page)
    index = oquest.select_pages(q, lo, hi, dones, done, pages)
    mask = None if attention_mask is None else attention_mask[..., : k.shape[2]].numpy()
    out = oquest.quest_reference(q, k, v, mask, scaling, index, dones, page)
    return torch.from_numpy(out).to(query.dtype), None


def test_golden_model_gives_the_reference_logits() -> None:
    held_out = _tokens(2, 2, 24)
    with torch.no_grad():
        logits = golden_model()(held_out).logits.float()
    torch.testing.assert_close(logits, torch.from_numpy(GOLDEN["dense_logits"]), atol=1e-3, rtol=1e-3)


def test_fp8_round_trip_gives_the_reference_tokens() -> None:
    cache = Cache(layers=[FP8Layer() for _ in range(6)])
    assert greedy(golden_model(), cache) == GOLDEN["kv_fp8_tokens"].tolist()


def test_kivi_gives_the_reference_tokens() -> None:
    cache = Cache(layers=[KIVILayer(2, 4, 8) for _ in range(6)])
    assert greedy(golden_model(), cache) == GOLDEN["kv_kivi_2bit_tokens"].tolist()


def test_quest_gives_the_reference_tokens() -> None:
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface

    AttentionInterface.register("quest_golden", quest_forward)
    AttentionMaskInterface.register("quest_golden", AttentionMaskInterface._global_mapping["sdpa"])
    # token_budget 32 over 16-token pages: 32 // 16 - 1 = 1 page besides the tail (quest/technique.py:99-106)
    cache = Cache(layers=[QuestLayer(16, 1) for _ in range(6)])
    assert greedy(golden_model("quest_golden"), cache) == GOLDEN["kv_quest_tokens"].tolist()
