"""KIVI's simulated storage on the GPU (``eco_kivi_fake_quantize``) against the oracle's quantize, bit for bit:
keys per channel over token groups and values per token over channel groups, at 2 / 4 / 8 bits, the group sizes the
reference's kernel tests use (tests/unit/test_attention_kivi.py:287-348: 16, 24, 32, 128) and a tiny one, head dims
48 / 64 / 128 (a value group that does not divide the head covers the whole head, kivi.py:143-154), bf16 / fp16 /
fp32 buffers; only the slots asked for change; scales beyond fp16 stay fp32; a group holding NaN becomes NaN."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kivi as okivi

pytestmark = pytest.mark.gpu


def expected(buffer: torch.Tensor, start: int, stop: int, bits: int, group: int, kind: str) -> np.ndarray:
    """The buffer after the reference's in-place quantization: fake_quantize rounded to the buffer's dtype."""
    x = buffer.float().cpu().numpy().copy()
    block = x[:, :, start:stop]
    b, h, t, d = block.shape
    if kind == "k":
        fq = okivi.fake_quantize(block.reshape(b, h, t // group, group, d), bits, axis=3)
    else:
        g = group if d % group == 0 else d
        fq = okivi.fake_quantize(block.reshape(b, h, t, d // g, g), bits, axis=4)
    x[:, :, start:stop] = torch.from_numpy(fq.reshape(block.shape)).to(buffer.dtype).float().numpy()
    return x


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("group,head_dim", [(4, 48), (16, 64), (24, 48), (32, 128), (128, 128), (32, 48)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fake_quantization_matches_the_oracle(bits, group, head_dim, dtype) -> None:
    from economize_amd.kivi import kivi_fake_quantize

    gen = torch.Generator().manual_seed(bits * 1000 + group * 10 + head_dim)
    full = (torch.randn(2, 3, 3 * group + 40, head_dim, generator=gen) * 3).to(dtype)
    full[..., 5] *= 20  # an outlier channel
    start, stop = group, 3 * group
    for kind in ("k", "v"):
        buffer = full.cuda()
        kivi_fake_quantize(buffer, start, stop, bits, group, kind)
        want = expected(full, start, stop, bits, group, kind)
        assert np.array_equal(buffer.float().cpu().numpy(), want), kind


def test_scales_beyond_fp16_and_nan_groups() -> None:
    from economize_amd.kivi import kivi_fake_quantize

    gen = torch.Generator().manual_seed(5)
    full = torch.randn(1, 2, 64, 64, generator=gen)
    full[0, 0, :32, 3] *= 1e7  # a key group whose scale and zero point stay fp32
    full[0, 1, 40, 9] = float("nan")  # the keys of channel 9 over tokens 32..63 of head 1, the values of token 40
    for kind in ("k", "v"):
        buffer = full.cuda()
        kivi_fake_quantize(buffer, 0, 64, 2, 32, kind)
        got = buffer.cpu().numpy()
        want = expected(full, 0, 64, 2, 32, kind)
        assert np.array_equal(np.isnan(got), np.isnan(want)), kind
        assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)]), kind
    assert np.isnan(expected(full, 0, 64, 2, 32, "k")[0, 1, 32:, 9]).all()


def test_refusals() -> None:
    from economize_amd.errors import ConfigError
    from economize_amd.kivi import kivi_fake_quantize

    buffer = torch.zeros(1, 1, 64, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ConfigError, match="whole groups"):
        kivi_fake_quantize(buffer, 0, 30, 2, 32, "k")
    with pytest.raises(ConfigError, match="out of the buffer"):
        kivi_fake_quantize(buffer, 32, 96, 2, 32, "k")
    with pytest.raises(ConfigError, match="bits"):
        kivi_fake_quantize(buffer, 0, 32, 3, 32, "k")
