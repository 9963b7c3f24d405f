"""The paged KIVI cache of the MI355X path, restated on the CPU (oracle).

The reference keeps KIVI codes either contiguous per row (``KIVIPacked``, attention/kivi.py:80-120) or in vLLM cells
that interleave a token's dense K/V with its codes (backends/vllm/kivi/layout.py:1-21). The MI355X path pages the
quantized part of every row in 32-token pages with one contiguous block per (page, KV head), laid out so that a
matrix-core operand is one vector load:

* key codes, token-major: ``[32 tokens][D * bits / 8 bytes]``, every token's channels packed in order;
* value codes, channel-major in 32-bit words: word ``(u * 16 + n) * (D / 16) + nd`` holds the codes of channel
  ``16 nd + n`` for tokens ``u * 32 / bits ..`` (``32 / bits`` tokens), so that the words a lane reads for its
  16-channel lane position are contiguous;
* key scales and zero points, fp16 ``[32 / G rows][D]`` each (one row per key group of ``G`` tokens);
* value scales and zero points, fp16 ``[D / G groups][32 tokens]`` each.

Codes are packed in 32-bit words: a word holds ``32 / bits`` elements (channels of a key, tokens of a value
channel), element ``e`` in byte ``e % 4`` at bit offset ``(e // 4) * bits``. Zero-extended to a byte, a code ``c < 16``
is the e4m3 bit pattern of ``c * 2**-9``, so the kernels turn a word into eight exact fp16 operands with two masks
and four conversions. This is a permutation of the reference's byte order (``pack_codes``, attention/kivi.py:38-45):
the codes themselves are the reference's (:func:`oracle.kivi.quantize`).

The full-precision residual of every row is a ring of ``W`` slots, token ``t`` at slot ``t % W``: keys
``[B, Hkv, W, D]`` (token-major), values ``[B, Hkv, D, W]`` (channel-major), bf16, like the reference's
``key_ring`` / ``value_ring`` (attention/kivi.py:100-108).

Pinned by (``tests/test_oracle_kivi_paged.py``): :func:`pack_words` / :func:`unpack_words` identity and the bit
position of single codes against the definition above written per element; block offsets against sizes; the codes,
scales and zero points inside a block against :func:`oracle.kivi.quantize_keys` / ``quantize_values`` (which the
reference's closed-form tests pin).
"""

from __future__ import annotations

import numpy as np

from .kivi import quantize_keys, quantize_values
from .numerics import round_bf16

__all__ = ["PAGE", "block_layout", "dense_view", "pack_words", "unpack_words", "value_codes", "value_words",
           "write_keys", "write_values"]

#: Tokens per KIVI page.
PAGE = 32


def pack_words(codes: np.ndarray, bits: int) -> np.ndarray:
    """Integer codes ``[..., n]`` (``n`` a multiple of ``32 / bits``) packed into bytes ``[..., n * bits / 8]``:
    element ``e`` of every word in byte ``e % 4`` at bit ``(e // 4) * bits``."""
    per_word = 32 // bits
    c = np.asarray(codes).astype(np.int64)
    if c.shape[-1] % per_word:
        raise ValueError(f"{c.shape[-1]} codes do not fill whole words of {per_word}")
    words = c.reshape(*c.shape[:-1], c.shape[-1] // per_word, per_word)
    out = np.zeros((*words.shape[:-1], 4), dtype=np.int64)
    for e in range(per_word):
        out[..., e % 4] |= words[..., e] << ((e // 4) * bits)
    return out.astype(np.uint8).reshape(*c.shape[:-1], c.shape[-1] * bits // 8)


def unpack_words(packed: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of :func:`pack_words` (``int32`` codes)."""
    per_word = 32 // bits
    p = np.asarray(packed).astype(np.int64)
    words = p.reshape(*p.shape[:-1], p.shape[-1] // 4, 4)
    out = np.zeros((*words.shape[:-1], per_word), dtype=np.int64)
    for e in range(per_word):
        out[..., e] = (words[..., e % 4] >> ((e // 4) * bits)) & ((1 << bits) - 1)
    return out.reshape(*p.shape[:-1], p.shape[-1] * 8 // bits).astype(np.int32)


def block_layout(head_dim: int, bits: int, group: int) -> dict[str, int]:
    """Byte offsets and size of one (page, KV head) block."""
    kc = PAGE * head_dim * bits // 8
    vc = head_dim * PAGE * bits // 8
    ks = (PAGE // group) * head_dim * 2
    vs = (head_dim // group) * PAGE * 2
    off = {"k_codes": 0, "v_codes": kc}
    off["k_scale"] = kc + vc
    off["k_zero"] = off["k_scale"] + ks
    off["v_scale"] = off["k_zero"] + ks
    off["v_zero"] = off["v_scale"] + vs
    off["size"] = off["v_zero"] + vs
    return off


def _half_bytes(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return np.ascontiguousarray(np.asarray(x, dtype=np.float32).astype(np.float16)).view(np.uint8)


def write_keys(blocks: np.ndarray, keys: np.ndarray, b: int, start: int, stop: int, table: np.ndarray, bits: int,
               group: int) -> None:
    """Quantize keys ``start:stop`` (whole pages) of row ``b`` of ``keys`` ``[B, Hkv, S, D]`` (float32 holding the
    bf16 values) into ``blocks`` ``[pages, Hkv, size]`` (``uint8``) through the block table."""
    _, heads, _, dim = keys.shape
    lay = block_layout(dim, bits, group)
    for p0 in range(start, stop, PAGE):
        page = table[b, p0 // PAGE]
        _, scale, zero, _ = quantize_keys(keys[b:b + 1], p0, p0 + PAGE, bits, group)  # [1, H, 32/G, D]
        codes = _key_codes(keys[b:b + 1], p0, bits, group)  # [H, 32, D]
        for h in range(heads):
            blk = blocks[page, h]
            blk[lay["k_codes"]:lay["v_codes"]] = pack_words(codes[h], bits).reshape(-1)
            blk[lay["k_scale"]:lay["k_zero"]] = _half_bytes(scale[0, h]).reshape(-1)
            blk[lay["k_zero"]:lay["v_scale"]] = _half_bytes(zero[0, h]).reshape(-1)


def _key_codes(keys: np.ndarray, p0: int, bits: int, group: int) -> np.ndarray:
    from .kivi import quantize

    block = np.asarray(keys[0, :, p0:p0 + PAGE], dtype=np.float32)  # [H, 32, D]
    h, t, d = block.shape
    codes, _, _ = quantize(block.reshape(h, t // group, group, d), bits, axis=2)
    return codes.reshape(h, t, d).astype(np.int64)


def value_words(codes: np.ndarray, bits: int) -> np.ndarray:
    """Value codes ``[D, 32]`` (channel, token) of one page laid out as the block's value-code bytes."""
    dim = codes.shape[0]
    tpw = 32 // bits
    nd = dim // 16
    words = np.zeros((bits, 16, nd, tpw), np.int64)  # [u, n, nd, token in word]
    for u in range(bits):
        for n in range(16):
            for j in range(nd):
                words[u, n, j] = codes[16 * j + n, u * tpw:(u + 1) * tpw]
    return pack_words(words.reshape(bits * 16 * nd, tpw), bits).reshape(-1)


def value_codes(raw: np.ndarray, dim: int, bits: int) -> np.ndarray:
    """Inverse of :func:`value_words`: codes ``[D, 32]`` of a block's value-code bytes."""
    tpw = 32 // bits
    nd = dim // 16
    words = unpack_words(raw.reshape(bits * 16 * nd, 4), bits).reshape(bits, 16, nd, tpw)
    codes = np.zeros((dim, PAGE), np.int64)
    for u in range(bits):
        for n in range(16):
            for j in range(nd):
                codes[16 * j + n, u * tpw:(u + 1) * tpw] = words[u, n, j]
    return codes


def write_values(blocks: np.ndarray, values: np.ndarray, b: int, start: int, stop: int, table: np.ndarray,
                 bits: int, group: int) -> None:
    """Quantize values ``start:stop`` (any tokens) of row ``b`` of ``values`` ``[B, Hkv, S, D]`` into ``blocks``:
    per token over groups of ``group`` channels; codes of the page's other tokens are kept."""
    _, heads, _, dim = values.shape
    lay = block_layout(dim, bits, group)
    _, scale, zero, _ = quantize_values(values[b:b + 1], start, stop, bits, group)  # [1, H, T, D/G]
    from .kivi import quantize

    block = np.asarray(values[b, :, start:stop], dtype=np.float32)  # [H, T, D]
    codes, _, _ = quantize(block.reshape(heads, stop - start, dim // group, group), bits, axis=3)
    codes = codes.reshape(heads, stop - start, dim).astype(np.int64)
    for t in range(start, stop):
        page = table[b, t // PAGE]
        pos = t % PAGE
        for h in range(heads):
            blk = blocks[page, h]
            vc = value_codes(blk[lay["v_codes"]:lay["k_scale"]], dim, bits)  # [D, 32]
            vc[:, pos] = codes[h, t - start]
            blk[lay["v_codes"]:lay["k_scale"]] = value_words(vc, bits)
            vs = blk[lay["v_scale"]:lay["v_zero"]].view(np.float16).reshape(dim // group, PAGE).copy()
            vz = blk[lay["v_zero"]:lay["size"]].view(np.float16).reshape(dim // group, PAGE).copy()
            with np.errstate(over="ignore"):
                vs[:, pos] = scale[0, h, t - start].astype(np.float16)
                vz[:, pos] = zero[0, h, t - start].astype(np.float16)
            blk[lay["v_scale"]:lay["v_zero"]] = vs.view(np.uint8).reshape(-1)
            blk[lay["v_zero"]:lay["size"]] = vz.view(np.uint8).reshape(-1)


def dense_view(blocks: np.ndarray, table: np.ndarray, k_ring: np.ndarray, v_ring: np.ndarray, lens, kq, vq,
               bits: int, group: int, round_values: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """The keys and values ``[B, Hkv, max(lens), D]`` (float32 holding bf16 values) attention sees: keys below
    ``kq[b]`` and values below ``vq[b]`` dequantized as the reference's ``dequantize`` does (``code * scale + zero``
    in fp32, two roundings, then bf16; attention/kivi.py:56-76), the others from the rings (token ``t`` at slot
    ``t % W``). ``round_values=False`` leaves the dequantized values in fp32 (not the reference: the form of a value
    product that never rounds a dequantized value, to measure how far such a product is from the reference)."""
    batch, heads, w, dim = k_ring.shape
    lay = block_layout(dim, bits, group)
    smax = int(max(lens))
    keys = np.zeros((batch, heads, smax, dim), np.float32)
    values = np.zeros((batch, heads, smax, dim), np.float32)
    for b, n in enumerate(lens):
        for t in range(int(n)):
            page, pos = table[b, t // PAGE], t % PAGE
            for h in range(heads):
                blk = blocks[page, h]
                if t < kq[b]:
                    codes = unpack_words(blk[lay["k_codes"]:lay["v_codes"]].reshape(PAGE, -1), bits)[pos]
                    s = blk[lay["k_scale"]:lay["k_zero"]].view(np.float16).reshape(-1, dim)[pos // group]
                    z = blk[lay["k_zero"]:lay["v_scale"]].view(np.float16).reshape(-1, dim)[pos // group]
                    keys[b, h, t] = round_bf16(((codes * s.astype(np.float32)).astype(np.float32)
                                                + z.astype(np.float32)).astype(np.float32))
                else:
                    keys[b, h, t] = k_ring[b, h, t % w]
                if t < vq[b]:
                    codes = value_codes(blk[lay["v_codes"]:lay["k_scale"]], dim, bits)[:, pos]
                    s = blk[lay["v_scale"]:lay["v_zero"]].view(np.float16).reshape(-1, PAGE)[:, pos]
                    z = blk[lay["v_zero"]:lay["size"]].view(np.float16).reshape(-1, PAGE)[:, pos]
                    s = np.repeat(s.astype(np.float32), group)
                    z = np.repeat(z.astype(np.float32), group)
                    v = ((codes * s).astype(np.float32) + z).astype(np.float32)
                    values[b, h, t] = round_bf16(v) if round_values else v
                else:
                    values[b, h, t] = v_ring[b, h, :, t % w]
    return keys, values
