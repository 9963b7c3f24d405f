"""The vLLM KIVI cell oracle pinned on the CPU against the already pinned KIVI quantize (the reference's
test_vllm_kivi.py:120-141 check: the cells hold economize's KIVI numbers) and the layout's stated byte positions
(backends/vllm/kivi/layout.py:1-21, 133-213)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kivi as okivi
from oracle import vllm_cells as oc
from oracle.numerics import round_bf16, round_fp16

ROUND = {"bf16": round_bf16, "f16": round_fp16, "f32": lambda x: np.asarray(x, np.float32)}
ES = {"bf16": 2, "f16": 2, "f32": 4}


def states(heads, tokens, dim, dtype, seed):
    rng = np.random.default_rng(seed)
    k = ROUND[dtype]((rng.standard_normal((heads, tokens, dim)) * 3).astype(np.float32))
    v = ROUND[dtype]((rng.standard_normal((heads, tokens, dim)) * 3).astype(np.float32))
    return k, v


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("bits,group,dim", [(2, 32, 128), (4, 16, 64), (8, 32, 64), (2, 32, 16), (4, 64, 128)])
def test_cells_hold_the_kivi_numbers(dtype, bits, group, dim) -> None:
    k, v = states(2, 4 * group + 5, dim, dtype, seed=bits * group + dim)
    layout = oc.cell_layout(dim, ES[dtype], bits, group)
    kq, vq = 3 * group, 3 * group + 2
    cells = oc.write_cells(k, v, kq, vq, layout, dtype)
    keys, values = oc.read_cells(cells, layout, dtype)
    vg = group if dim % group == 0 else dim
    want_k = k.copy()
    want_k[:, :kq] = ROUND[dtype](okivi.fake_quantize(k[:, :kq].reshape(2, kq // group, group, dim), bits, axis=2)
                                  .reshape(2, kq, dim))
    want_v = v.copy()
    want_v[:, :vq] = ROUND[dtype](okivi.fake_quantize(v[:, :vq].reshape(2, vq, dim // vg, vg), bits, axis=3)
                                  .reshape(2, vq, dim))
    assert np.array_equal(keys, want_k) and np.array_equal(values, want_v)
    # the dense entries hold the same numbers (so vLLM's own kernels attend over them too)
    dense_k = oc._from_dtype(cells[:, :, :layout.off_v], dtype)
    assert np.array_equal(dense_k, want_k)
    # flags: quantized cells 1, the rest 0; the cells past the quantized prefix are the dense states only
    assert (cells[:, :kq, layout.off_flag] == 1).all() and (cells[:, kq:, layout.off_flag] == 0).all()
    assert (cells[:, :vq, layout.off_flag + 1] == 1).all() and (cells[:, vq:, layout.off_flag + 1] == 0).all()
    assert (cells[:, vq:, layout.off_vs:] == 0).all() if vq >= kq else True


def test_aux_entries_and_codes_sit_where_the_layout_says() -> None:
    """Entry e of the key group starting at s0 is in the cell of token s0 + e // ka at aux slot e % ka (D scales,
    then D zero points); code of channel j pb + i is bits i * bits of code byte j."""
    dim, group, bits = 64, 16, 4
    layout = oc.cell_layout(dim, 2, bits, group)
    assert layout.key_aux == 8 and layout.value_group == 16
    k, v = states(1, 2 * group, dim, "bf16", seed=5)
    cells = oc.write_cells(k, v, 2 * group, 0, layout, "bf16")
    codes, scale, low = okivi.quantize(k[:, :2 * group].reshape(1, 2, group, dim), bits, axis=2)
    for grp in range(2):
        s0 = grp * group
        entries = np.concatenate([scale[0, grp, 0], low[0, grp, 0]]).astype(np.float16)
        for e in range(2 * dim):
            cell = cells[0, s0 + e // layout.key_aux]
            at = layout.off_ka + 2 * (e % layout.key_aux)
            assert cell[at: at + 2].view(np.float16)[0] == entries[e], (grp, e)
        for t in range(group):
            for ch in range(dim):
                byte = cells[0, s0 + t, layout.off_kc + ch // 2]
                assert (byte >> (4 * (ch % 2))) & 15 == int(codes[0, grp, t, ch])


def test_offsets_have_the_closed_form() -> None:
    layout = oc.cell_layout(128, 2, 2, 32)  # bf16, int2, groups of 32
    assert (layout.off_v, layout.off_vs, layout.off_vz, layout.off_ka) == (256, 512, 520, 528)
    assert (layout.key_aux, layout.off_kc, layout.off_vc, layout.off_flag, layout.size) == (8, 544, 576, 608, 624)
    assert oc.cell_layout(16, 4, 2, 32).value_group == 16  # a value group that does not divide the head covers it


def test_a_scale_beyond_fp16_sets_the_overflow_flag() -> None:
    k, v = states(1, 64, 32, "f32", seed=2)
    k[0, :32, 3] *= 1e6
    layout = oc.cell_layout(32, 4, 2, 32)
    cells = oc.write_cells(k, v, 64, 0, layout, "f32")
    assert (cells[0, :32, layout.off_flag] == oc.FLAG_OVERFLOW).all()
    assert (cells[0, 32:, layout.off_flag] == oc.FLAG_PACKED).all()
    keys, _ = oc.read_cells(cells, layout, "f32")
    want = okivi.fake_quantize(k[:, :32].reshape(1, 1, 32, 32), 2, axis=2).reshape(1, 32, 32)
    assert np.array_equal(keys[:, :32], want)  # an overflowed group is read from its dense entries
