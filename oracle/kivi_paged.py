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
position of single codes, element by element; :func:`value_words` / :func:`value_codes` identity and the word and bit
of single codes against the word formula above; block offsets against sizes; :func:`dense_view` of pages written by
:func:`write_keys` / :func:`write_values` against :func:`oracle.kivi.dequantize` of the contiguous codes of
:func:`oracle.kivi.quantize_keys` / ``quantize_values`` (the reference's ``KIVIPacked`` format, which the
reference's closed-form tests pin), rounded to bf16, and values written in several ranges against one write.
"""

from __future__ import annotations

import numpy as np

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


def value_words(codes: np.ndarray, bits: int) -> np.ndarray:
    """Value codes ``[..., D, 32]`` (channel, token) of pages laid out as the blocks' value-code bytes
    ``[..., D * 32 * bits / 8]``: word ``(u * 16 + n) * (D / 16) + nd`` holds channel ``16 nd + n``, tokens
    ``u * 32 / bits ..`` (``32 / bits`` of them)."""
    c = np.asarray(codes).astype(np.int64)
    *lead, dim, tokens = c.shape
    tpw = 32 // bits
    nd = dim // 16
    # [..., nd, n, u, e] -> [..., u, n, nd, e]
    w = c.reshape(*lead, nd, 16, bits, tpw)
    k = len(lead)
    w = np.moveaxis(w, [k, k + 1, k + 2], [k + 2, k + 1, k])
    return pack_words(w.reshape(*lead, bits * 16 * nd * tpw), bits)


def value_codes(raw: np.ndarray, dim: int, bits: int) -> np.ndarray:
    """Inverse of :func:`value_words`: codes ``[..., D, 32]`` of value-code bytes ``[..., D * 32 * bits / 8]``."""
    r = np.asarray(raw)
    lead = r.shape[:-1]
    tpw = 32 // bits
    nd = dim // 16
    k = len(lead)
    w = unpack_words(r, bits).reshape(*lead, bits, 16, nd, tpw)
    w = np.moveaxis(w, [k, k + 1, k + 2], [k + 2, k + 1, k])  # [..., nd, n, u, e]
    return w.reshape(*lead, dim, PAGE).astype(np.int64)


def _rows_pages(table: np.ndarray, b: int, first: int, count: int) -> np.ndarray:
    return np.asarray(table[b, first:first + count]).astype(np.int64)


def write_keys(blocks: np.ndarray, keys: np.ndarray, b: int, start: int, stop: int, table: np.ndarray, bits: int,
               group: int) -> None:
    """Quantize keys ``start:stop`` (whole pages) of row ``b`` of ``keys`` ``[B, Hkv, S, D]`` (float32 holding the
    bf16 values) into ``blocks`` ``[pages, Hkv, size]`` (``uint8``) through the block table: per channel over groups
    of ``group`` tokens (:func:`oracle.kivi.quantize`)."""
    from .kivi import quantize

    if stop <= start:
        return
    _, heads, _, dim = keys.shape
    lay = block_layout(dim, bits, group)
    block = np.asarray(keys[b, :, start:stop], dtype=np.float32)  # [H, T, D]
    t = block.shape[1]
    npg = t // PAGE
    codes, scale, low = quantize(block.reshape(heads, t // group, group, dim), bits, axis=2)
    codes = codes.reshape(heads, npg, PAGE, dim).astype(np.int64)
    scale = scale.reshape(heads, npg, PAGE // group, dim)
    low = low.reshape(heads, npg, PAGE // group, dim)
    pages = _rows_pages(table, b, start // PAGE, npg)
    kc = pack_words(codes, bits).reshape(heads, npg, -1)
    blocks[pages, :, lay["k_codes"]:lay["v_codes"]] = kc.transpose(1, 0, 2)
    blocks[pages, :, lay["k_scale"]:lay["k_zero"]] = _half_bytes(scale).reshape(heads, npg, -1).transpose(1, 0, 2)
    blocks[pages, :, lay["k_zero"]:lay["v_scale"]] = _half_bytes(low).reshape(heads, npg, -1).transpose(1, 0, 2)


def write_values(blocks: np.ndarray, values: np.ndarray, b: int, start: int, stop: int, table: np.ndarray,
                 bits: int, group: int) -> None:
    """Quantize values ``start:stop`` (any tokens) of row ``b`` of ``values`` ``[B, Hkv, S, D]`` into ``blocks``:
    per token over groups of ``group`` channels; codes of the pages' other tokens are kept."""
    from .kivi import quantize

    if stop <= start:
        return
    _, heads, _, dim = values.shape
    lay = block_layout(dim, bits, group)
    block = np.asarray(values[b, :, start:stop], dtype=np.float32)  # [H, T, D]
    t = block.shape[1]
    codes, scale, low = quantize(block.reshape(heads, t, dim // group, group), bits, axis=3)
    codes = codes.reshape(heads, t, dim).astype(np.int64)
    scale, low = scale.reshape(heads, t, dim // group), low.reshape(heads, t, dim // group)
    for p0 in range(start - start % PAGE, stop, PAGE):
        page = int(table[b, p0 // PAGE])
        lo, hi = max(start, p0), min(stop, p0 + PAGE)
        blk = blocks[page]  # [H, size]
        vc = value_codes(blk[:, lay["v_codes"]:lay["k_scale"]], dim, bits)  # [H, D, 32]
        vc[:, :, lo - p0:hi - p0] = codes[:, lo - start:hi - start].transpose(0, 2, 1)
        blk[:, lay["v_codes"]:lay["k_scale"]] = value_words(vc, bits)
        vs = blk[:, lay["v_scale"]:lay["v_zero"]].copy().view(np.float16).reshape(heads, dim // group, PAGE)
        vz = blk[:, lay["v_zero"]:lay["size"]].copy().view(np.float16).reshape(heads, dim // group, PAGE)
        with np.errstate(over="ignore"):
            vs[:, :, lo - p0:hi - p0] = scale[:, lo - start:hi - start].transpose(0, 2, 1).astype(np.float16)
            vz[:, :, lo - p0:hi - p0] = low[:, lo - start:hi - start].transpose(0, 2, 1).astype(np.float16)
        blk[:, lay["v_scale"]:lay["v_zero"]] = vs.view(np.uint8).reshape(heads, -1)
        blk[:, lay["v_zero"]:lay["size"]] = vz.view(np.uint8).reshape(heads, -1)


def dense_view(blocks: np.ndarray, table: np.ndarray, k_ring: np.ndarray, v_ring: np.ndarray, lens, kq, vq,
               bits: int, group: int, rows=None) -> tuple[np.ndarray, np.ndarray]:
    """The keys and values ``[B, Hkv, max(lens), D]`` (float32 holding bf16 values) attention sees: keys below
    ``kq[b]`` and values below ``vq[b]`` dequantized as the reference's ``dequantize`` does (``code * scale + zero``
    in fp32, two roundings, then bf16; attention/kivi.py:56-76), the others from the rings (token ``t`` at slot
    ``t % W``). ``rows`` limits the work to those batch rows (the others stay zero)."""
    batch, heads, w, dim = k_ring.shape
    lay = block_layout(dim, bits, group)
    smax = int(max(lens))
    keys = np.zeros((batch, heads, smax, dim), np.float32)
    values = np.zeros((batch, heads, smax, dim), np.float32)
    for b in (range(batch) if rows is None else rows):
        n = int(lens[b])
        if n <= 0:
            continue
        npg = (n + PAGE - 1) // PAGE
        blk = blocks[_rows_pages(table, b, 0, npg)]  # [P, H, size]
        kc = unpack_words(blk[:, :, lay["k_codes"]:lay["v_codes"]].reshape(npg, heads, PAGE, -1), bits)
        ks = blk[:, :, lay["k_scale"]:lay["k_zero"]].copy().view(np.float16).reshape(npg, heads, PAGE // group, dim)
        kz = blk[:, :, lay["k_zero"]:lay["v_scale"]].copy().view(np.float16).reshape(npg, heads, PAGE // group, dim)
        ks = np.repeat(ks.astype(np.float32), group, axis=2)
        kz = np.repeat(kz.astype(np.float32), group, axis=2)
        kd = round_bf16(((kc * ks).astype(np.float32) + kz).astype(np.float32))  # [P, H, 32, D]
        kd = kd.transpose(1, 0, 2, 3).reshape(heads, npg * PAGE, dim)[:, :n]
        vc = value_codes(blk[:, :, lay["v_codes"]:lay["k_scale"]], dim, bits)  # [P, H, D, 32]
        vs = blk[:, :, lay["v_scale"]:lay["v_zero"]].copy().view(np.float16).reshape(npg, heads, dim // group, PAGE)
        vz = blk[:, :, lay["v_zero"]:lay["size"]].copy().view(np.float16).reshape(npg, heads, dim // group, PAGE)
        vs = np.repeat(vs.astype(np.float32), group, axis=2)
        vz = np.repeat(vz.astype(np.float32), group, axis=2)
        with np.errstate(invalid="ignore", over="ignore"):
            vd = round_bf16(((vc * vs).astype(np.float32) + vz).astype(np.float32))  # [P, H, D, 32]
        vd = vd.transpose(1, 0, 3, 2).reshape(heads, npg * PAGE, dim)[:, :n]
        slots = np.arange(n) % w
        kr = k_ring[b][:, slots]  # [H, n, D]
        vr = v_ring[b][:, :, slots].transpose(0, 2, 1)
        t = np.arange(n)[None, :, None]
        keys[b, :, :n] = np.where(t < kq[b], kd, kr)
        values[b, :, :n] = np.where(t < vq[b], vd, vr)
    return keys, values
