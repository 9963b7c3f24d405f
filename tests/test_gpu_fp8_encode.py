"""The dense fp8 encode kernel (``eco_fp8_encode``) against the oracle's fp8_encode and token_scale
(techniques/kv_quant/fp8.py:81-97), bit for bit: codes of every scale mode (none, per head, per token) in both
formats, from bf16 / fp16 / fp32 states, into a strided cache buffer; the per-token scales themselves; NaN, infinities
and saturation."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu

FORMATS = {torch.float8_e4m3fn: "e4m3", torch.float8_e5m2: "e5m2"}


def states(shape, dtype, seed: int, specials: bool = False) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=gen) * torch.exp2(torch.randint(-12, 12, shape, generator=gen).float())
    if specials:
        flat = x.view(-1)
        flat[:6] = torch.tensor([float("nan"), float("inf"), -float("inf"), 1e9, -1e9, 0.0])
    return x.to(dtype)


def codes_of(buffer: torch.Tensor) -> np.ndarray:
    return buffer.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("dtype", list(FORMATS))
@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("head_dim", [16, 100, 128, 256, 456, 512])
def test_unscaled_and_per_head_codes_match_the_oracle(dtype, in_dtype, head_dim) -> None:
    from economize_amd.fp8 import fp8_encode

    x = states((2, 3, 37, head_dim), in_dtype, seed=head_dim, specials=True)
    ref_in = x.float().numpy()
    fmt = FORMATS[dtype]
    buffer = torch.full((2, 3, 50, head_dim), 0x55, dtype=torch.uint8).cuda().view(dtype)
    got = fp8_encode(x.cuda(), dtype, buffer[:, :, 5:42])
    assert np.array_equal(codes_of(got), ofp8.fp8_encode(ref_in, fmt, None))
    assert (codes_of(buffer)[:, :, :5] == 0x55).all() and (codes_of(buffer)[:, :, 42:] == 0x55).all()
    scale = torch.tensor([0.5, 3.0, 1e-3])
    got = fp8_encode(x.cuda(), dtype, head_scale=scale.cuda())
    assert np.array_equal(codes_of(got), ofp8.fp8_encode(ref_in, fmt, scale.numpy().reshape(1, 3, 1, 1)))


@pytest.mark.parametrize("dtype", list(FORMATS))
@pytest.mark.parametrize("head_dim", [16, 64, 200, 512])
def test_per_token_scales_and_codes_match_the_oracle(dtype, head_dim) -> None:
    """token_scale's rule (absmax / format max, at least 1e-12) written beside the codes, for finite rows, an
    all-zero row and rows of huge values."""
    from economize_amd.fp8 import fp8_encode

    x = states((2, 4, 29, head_dim), torch.bfloat16, seed=7 + head_dim)
    x[0, 1, 3] = 0.0
    x[1, 2, 5] *= 1e30
    fmt = FORMATS[dtype]
    scales = torch.full((2, 4, 40), -1.0).cuda()
    got = fp8_encode(x.cuda(), dtype, token_scale=scales[:, :, 4:33])
    want_scale = ofp8.token_scale(x.float().numpy(), fmt)
    assert np.array_equal(scales[:, :, 4:33].cpu().numpy(), want_scale[..., 0])
    assert (scales[:, :, :4] == -1).all() and (scales[:, :, 33:] == -1).all()
    assert np.array_equal(codes_of(got), ofp8.fp8_encode(x.float().numpy(), fmt, want_scale))


def test_a_nan_row_has_a_nan_token_scale() -> None:
    """torch's amax propagates NaN, so the reference's per-token scale of a row holding NaN is NaN and every code of
    the row is NaN (fp8.py:95-97)."""
    from economize_amd.fp8 import fp8_encode

    x = states((1, 2, 3, 64), torch.float32, seed=3)
    x[0, 1, 2, 7] = float("nan")
    scales = torch.empty(1, 2, 3).cuda()
    got = codes_of(fp8_encode(x.cuda(), torch.float8_e4m3fn, token_scale=scales))
    assert torch.isnan(scales[0, 1, 2]) and not torch.isnan(scales[0, :, :2]).any()
    assert ((got[0, 1, 2] & 0x7F) == 0x7F).all()  # e4m3fn NaN, either sign
    assert np.array_equal(got[0, :, :2], ofp8.fp8_encode(x[0, :, :2].numpy(), "e4m3",
                                                         ofp8.token_scale(x[0, :, :2].numpy(), "e4m3")))


def test_refusals() -> None:
    from economize_amd.errors import ConfigError
    from economize_amd.fp8 import fp8_encode

    x = torch.zeros(1, 2, 3, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ConfigError):
        fp8_encode(x, torch.bfloat16)
    with pytest.raises(ConfigError, match="head scales"):
        fp8_encode(x, torch.float8_e4m3fn, head_scale=torch.ones(3, device="cuda"))
    with pytest.raises(ConfigError, match="token_scale"):
        fp8_encode(x, torch.float8_e4m3fn, token_scale=torch.ones(1, 2, 4, device="cuda"))
    with pytest.raises(ConfigError, match="exclude"):
        fp8_encode(x, torch.float8_e4m3fn, head_scale=torch.ones(2, device="cuda"),
                   token_scale=torch.ones(1, 2, 3, device="cuda"))
