"""The C ABI's KIVI cell layout (``eco_kivi_cells_layout``, a host computation) equals the oracle's
(backends/vllm/kivi/layout.py:133-213) for every head size, dtype, bits and group it takes, and refuses the rest."""

from __future__ import annotations

import pytest
import torch

from economize_amd.errors import ConfigError
from oracle import vllm_cells as oc


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_layout_matches_the_oracle(dtype) -> None:
    from economize_amd.vllm_kivi import cell_layout

    es = torch.empty((), dtype=dtype).element_size()
    for head in (16, 32, 64, 128, 256):
        for bits in (2, 4, 8):
            for group in (1, 2, 8, 16, 32, 64, 128):
                got = cell_layout(head, dtype, bits, group)
                want = oc.cell_layout(head, es, bits, group)
                for name in ("value_group", "key_aux", "off_v", "off_vs", "off_vz", "off_ka", "off_kc", "off_vc",
                             "off_flag", "size"):
                    assert getattr(got, name) == getattr(want, name), (head, bits, group, name)


def test_layout_refusals() -> None:
    from economize_amd.vllm_kivi import cell_layout

    for args in ((48, torch.bfloat16, 2, 32), (128, torch.bfloat16, 3, 32), (128, torch.bfloat16, 2, 24),
                 (512, torch.bfloat16, 2, 32), (128, torch.float8_e4m3fn, 2, 32)):
        with pytest.raises(ConfigError):
            cell_layout(*args)
