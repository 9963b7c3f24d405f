"""Pins the oracle's paged KIVI layout (oracle/kivi_paged.py) independently of its own code paths.

* ``pack_words`` / ``unpack_words``: identity, and a single code lands in byte ``e % 4`` at bit ``(e // 4) * bits``
  of its word, element by element;
* ``value_words`` / ``value_codes``: identity, and a single code of channel ``d``, token ``t`` lands in word
  ``(u * 16 + n) * (D / 16) + nd`` (``d = 16 nd + n``, ``u = t // (32 / bits)``), element ``t % (32 / bits)``;
* ``block_layout``: the parts are contiguous and the sizes are the C library's;
* ``dense_view`` of pages written by ``write_keys`` / ``write_values`` equals ``oracle.kivi.dequantize`` of the
  contiguous codes, scales and zero points of ``quantize_keys`` / ``quantize_values`` (the reference's
  ``KIVIPacked`` format, attention/kivi.py:80-120, whose quantizer tests/test_oracle_kivi.py pins), and the rings
  above the quantized prefixes;
* values and keys written in several ranges give the same bytes as one write.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kivi as ok
from oracle import kivi_paged as okp
from oracle import paged as opaged
from oracle.numerics import round_bf16


@pytest.mark.parametrize("bits", [2, 4])
def test_words_identity_and_bit_positions(bits: int) -> None:
    per_word = 32 // bits
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 2**bits, (5, 3 * per_word))
    assert np.array_equal(okp.unpack_words(okp.pack_words(codes, bits), bits), codes)
    for e in range(per_word):
        for c in (1, 2**bits - 1):
            one = np.zeros(per_word, np.int64)
            one[e] = c
            packed = okp.pack_words(one, bits)
            want = np.zeros(4, np.uint8)
            want[e % 4] = c << ((e // 4) * bits)
            assert np.array_equal(packed, want), (e, c)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("dim", [64, 128])
def test_value_words_identity_and_positions(bits: int, dim: int) -> None:
    tpw = 32 // bits
    rng = np.random.default_rng(dim + bits)
    codes = rng.integers(0, 2**bits, (2, 3, dim, okp.PAGE))
    raw = okp.value_words(codes, bits)
    assert raw.shape == (2, 3, dim * okp.PAGE * bits // 8)
    assert np.array_equal(okp.value_codes(raw, dim, bits), codes)
    for d, t in [(0, 0), (5, 7), (17, 8), (dim - 1, 31), (33, 16), (16 * 3 + 9, 21)]:
        one = np.zeros((dim, okp.PAGE), np.int64)
        one[d, t] = 2**bits - 1
        got = okp.value_words(one, bits)
        nd, n, u, e = d // 16, d % 16, t // tpw, t % tpw
        word = (u * 16 + n) * (dim // 16) + nd
        want = np.zeros_like(got)
        want[4 * word + e % 4] = (2**bits - 1) << ((e // 4) * bits)
        assert np.array_equal(got, want), (d, t)


@pytest.mark.parametrize("bits,dim,size", [(2, 64, 1536), (4, 64, 2560), (2, 128, 3072), (4, 128, 5120)])
def test_block_layout(bits: int, dim: int, size: int) -> None:
    lay = okp.block_layout(dim, bits, 32)
    order = ["k_codes", "v_codes", "k_scale", "k_zero", "v_scale", "v_zero", "size"]
    lengths = [32 * dim * bits // 8, dim * 32 * bits // 8, 2 * dim, 2 * dim, 2 * dim, 2 * dim]
    assert lay["k_codes"] == 0
    for a, b, n in zip(order, order[1:], lengths):
        assert lay[b] - lay[a] == n
    assert lay["size"] == size


def test_block_size_is_the_libraries() -> None:
    """The C ABI's eco_kivi_block_bytes (a host function) agrees with the oracle's layout."""
    from economize_amd import _lib

    for bits in (2, 4):
        for dim in (64, 128):
            assert int(_lib.lib().eco_kivi_block_bytes(dim, bits, 32)) == okp.block_layout(dim, bits, 32)["size"]


def _rings(k, v, lens, w):
    batch, heads, _, dim = k.shape
    k_ring = np.zeros((batch, heads, w, dim), np.float32)
    v_ring = np.zeros((batch, heads, dim, w), np.float32)
    for b, n in enumerate(lens):
        for t in range(max(0, n - w), n):
            k_ring[b, :, t % w] = k[b, :, t]
            v_ring[b, :, :, t % w] = v[b, :, t]
    return k_ring, v_ring


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("dim", [64, 128])
def test_dense_view_equals_contiguous_dequantize(bits: int, dim: int) -> None:
    rng = np.random.default_rng(11 * bits + dim)
    lens = [300, 97, 161]
    batch, heads, smax, w = len(lens), 2, max(lens), 384
    k = round_bf16(rng.standard_normal((batch, heads, smax, dim)).astype(np.float32) * 3)
    v = round_bf16(rng.standard_normal((batch, heads, smax, dim)).astype(np.float32))
    kq = np.array([(n // 128) * 128 for n in lens])  # whole 32-token groups below kq
    vq = np.array([max(n - 128, 0) for n in lens])
    table, pages = opaged.shuffled_block_table(lens, okp.PAGE, seed=3)
    size = okp.block_layout(dim, bits, 32)["size"]
    blocks = np.zeros((pages, heads, size), np.uint8)
    for b in range(batch):
        okp.write_keys(blocks, k, b, 0, int(kq[b]), table, bits, 32)
        okp.write_values(blocks, v, b, 0, int(vq[b]), table, bits, 32)
    k_ring, v_ring = _rings(k, v, lens, w)
    keys, values = okp.dense_view(blocks, table, k_ring, v_ring, lens, kq, vq, bits, 32)
    for b, n in enumerate(lens):
        if kq[b]:
            packed, scale, zero, _ = ok.quantize_keys(k[b:b + 1], 0, int(kq[b]), bits, 32)
            want = ok.dequantize(packed, scale, zero, bits, "key", 32)[0]
            assert np.array_equal(keys[b, :, :kq[b]], want)
        if vq[b]:
            packed, scale, zero, _ = ok.quantize_values(v[b:b + 1], 0, int(vq[b]), bits, 32)
            want = ok.dequantize(packed, scale, zero, bits, "value", 32)[0]
            assert np.array_equal(values[b, :, :vq[b]], want)
        assert np.array_equal(keys[b, :, kq[b]:n], k[b, :, kq[b]:n])
        assert np.array_equal(values[b, :, vq[b]:n], v[b, :, vq[b]:n])
        assert not keys[b, :, n:].any() and not values[b, :, n:].any()


@pytest.mark.parametrize("bits", [2, 4])
def test_writes_in_ranges_equal_one_write(bits: int) -> None:
    rng = np.random.default_rng(bits)
    dim, heads, n = 128, 3, 200
    k = round_bf16(rng.standard_normal((1, heads, n, dim)).astype(np.float32))
    v = round_bf16(rng.standard_normal((1, heads, n, dim)).astype(np.float32))
    table, pages = opaged.shuffled_block_table([n], okp.PAGE, seed=7)
    size = okp.block_layout(dim, bits, 32)["size"]
    once = np.zeros((pages, heads, size), np.uint8)
    okp.write_keys(once, k, 0, 0, 192, table, bits, 32)
    okp.write_values(once, v, 0, 0, 173, table, bits, 32)
    parts = np.zeros_like(once)
    for a, b in [(0, 64), (64, 96), (96, 192)]:
        okp.write_keys(parts, k, 0, a, b, table, bits, 32)
    for a, b in [(0, 31), (31, 32), (32, 100), (100, 101), (101, 173)]:
        okp.write_values(parts, v, 0, a, b, table, bits, 32)
    assert np.array_equal(once, parts)
