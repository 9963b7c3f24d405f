"""The paged KV-cache layout of the fp8/bf16 paged path, its block tables and gathers (oracle).

The reference has no paged fp8 or paged Quest kernel; its paged KIVI cache (backends/vllm/kivi/layout.py:1-21) is
vLLM's. The fp8/bf16 paged path stores, per layer, two tensors in vLLM's original paged-attention layout:

* keys   ``[pages, Hkv, D / X, PAGE, X]`` with ``X = 16 / element bytes`` (16-byte runs of a token's channels);
* values ``[pages, Hkv, D, PAGE]`` (every channel's ``PAGE`` tokens contiguous).

Row ``b``'s token ``t`` lives in page ``block_table[b, t // PAGE]`` at position ``t % PAGE``; ``slot = page * PAGE +
position`` is the slot mapping of an append. Parity with the contiguous definitions is checked the way the
reference checks its paged kernel (tests/integrations/test_vllm_kivi_gpu.py:180-218 ``_hf_operands``): gather the
pages back into ``[B, Hkv, S, D]`` and run the contiguous definition.

``shuffled_block_table`` assigns every row ``ceil(len / PAGE)`` distinct pages from a seeded permutation (as
test_vllm_kivi_gpu.py:39-51 ``_pages``).

Pinned by (``tests/test_oracle_paged.py``): scatter followed by gather is the identity on every in-range slot,
every slot is written exactly once, and the element of (b, h, t, d) sits at the byte the layout formula names.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "gather_kv",
    "k_cache_shape",
    "scatter_kv",
    "shuffled_block_table",
    "slot_mapping",
    "v_cache_shape",
]


def k_cache_shape(pages: int, kv_heads: int, head_dim: int, page: int, element_bytes: int) -> tuple[int, ...]:
    x = 16 // element_bytes
    return (pages, kv_heads, head_dim // x, page, x)


def v_cache_shape(pages: int, kv_heads: int, head_dim: int, page: int) -> tuple[int, ...]:
    return (pages, kv_heads, head_dim, page)


def shuffled_block_table(seq_lens, page: int, seed: int, spare: int = 3) -> tuple[np.ndarray, int]:
    """``(block_table int32 [B, max pages], total pages)``: distinct pages per row from a seeded permutation, unused
    entries -1."""
    need = [-(-int(s) // page) for s in seq_lens]
    total = sum(need) + spare
    order = np.random.default_rng(seed).permutation(total)
    table = np.full((len(need), max(max(need), 1)), -1, dtype=np.int32)
    at = 0
    for b, n in enumerate(need):
        table[b, :n] = order[at: at + n]
        at += n
    return table, total


def slot_mapping(block_table: np.ndarray, b: int, start: int, count: int, page: int) -> np.ndarray:
    """Slots of row ``b``'s tokens ``start .. start + count - 1``."""
    t = np.arange(start, start + count)
    return (block_table[b, t // page].astype(np.int64) * page + t % page).astype(np.int32)


def scatter_kv(keys: np.ndarray, values: np.ndarray, seq_lens, block_table: np.ndarray, total_pages: int,
               page: int, element_bytes: int) -> tuple[np.ndarray, np.ndarray]:
    """The caches holding row ``b``'s first ``seq_lens[b]`` tokens of ``keys``/``values`` ``[B, Hkv, S, D]``
    (any element dtype: bytes, bf16 bit patterns or floats); untouched entries are 0."""
    _, h, _, d = keys.shape
    x = 16 // element_bytes
    kc = np.zeros(k_cache_shape(total_pages, h, d, page, element_bytes), dtype=keys.dtype)
    vc = np.zeros(v_cache_shape(total_pages, h, d, page), dtype=values.dtype)
    for b, n in enumerate(seq_lens):
        t = np.arange(int(n))
        pg, pos = block_table[b, t // page], t % page
        k = keys[b, :, : int(n)].reshape(h, int(n), d // x, x)  # [H, T, C, X]
        kc[pg, :, :, pos, :] = np.transpose(k, (1, 0, 2, 3))
        vc[pg, :, :, pos] = np.transpose(values[b, :, : int(n)], (1, 0, 2))
    return kc, vc


def gather_kv(k_cache: np.ndarray, v_cache: np.ndarray, block_table: np.ndarray, seq_lens, page: int
              ) -> tuple[np.ndarray, np.ndarray]:
    """``[B, Hkv, max(seq_lens), D]`` keys and values read back through the block table (0 past each row's
    length)."""
    _, h, c, _, x = k_cache.shape
    d = c * x
    smax = int(max(seq_lens))
    keys = np.zeros((len(seq_lens), h, smax, d), dtype=k_cache.dtype)
    values = np.zeros((len(seq_lens), h, smax, d), dtype=v_cache.dtype)
    for b, n in enumerate(seq_lens):
        t = np.arange(int(n))
        pg, pos = block_table[b, t // page], t % page
        k = k_cache[pg, :, :, pos, :]  # [T, H, C, X]
        keys[b, :, : int(n)] = np.transpose(k, (1, 0, 2, 3)).reshape(h, int(n), d)
        values[b, :, : int(n)] = np.transpose(v_cache[pg, :, :, pos], (1, 0, 2))
    return keys, values
