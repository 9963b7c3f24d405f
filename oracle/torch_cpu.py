"""The paged fp8 decode-attention call restated in torch on the CPU, fp32 (oracle; the CPU baseline).

This is the reference's CPU arithmetic for the call the kernel replaces, written with torch's CPU operators so that
it runs multithreaded: every row's pages gathered from the paged cache (``[pages, Hkv, D/16, 16, 16]`` keys,
``[pages, Hkv, D, 16]`` values), the bytes decoded as ``fp8_decode`` does with ``out=float32``
(``raw.view(fp8).float() * scale``, techniques/kv_quant/fp8.py:89-92), and the fp32 definition of
attention/decode.py:66-103 for one query per row (every held token visible): scores ``q . k * scale``, softmax,
``probs @ v``, grouped-query heads reading KV head ``h // G``.

Test infrastructure only: ``bench.py`` times it as the CPU baseline and compares its output with the GPU call's.
Pinned by (``tests/test_oracle_torch_cpu.py``): equality within fp32 rounding with :func:`oracle.attention.
reference_attention` over :func:`oracle.fp8.fp8_decode` of :func:`oracle.paged.gather_kv`'s gathered bytes, on
ragged rows with GQA.
"""

from __future__ import annotations

import torch

__all__ = ["paged_fp8_decode_attention"]


def paged_fp8_decode_attention(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, k_scale: torch.Tensor,
                               v_scale: torch.Tensor, block_table: torch.Tensor, lens: list[int], scale: float,
                               fmt: torch.dtype = torch.float8_e4m3fn) -> torch.Tensor:
    """``[B, 1, Hq, D]`` float32 attention of ``query`` ``[B, 1, Hq, D]`` over the paged cache (``keys`` / ``values``
    uint8 in the paged layout, per-head fp32 scales ``[Hkv]``, int block table ``[B, pages]``, row lengths)."""
    batch, _, q_heads, dim = query.shape
    kv_heads = keys.shape[1]
    groups = q_heads // kv_heads
    out = torch.zeros(batch, 1, q_heads, dim, dtype=torch.float32)
    ks = k_scale.float().reshape(kv_heads, 1, 1)
    vs = v_scale.float().reshape(kv_heads, 1, 1)
    for b, n in enumerate(lens):
        if n <= 0:
            continue
        pages = block_table[b, : (n + 15) // 16].long()
        k = keys[pages].permute(1, 0, 3, 2, 4).reshape(kv_heads, -1, dim)[:, :n]
        v = values[pages].permute(1, 0, 3, 2).reshape(kv_heads, -1, dim)[:, :n]
        kf = k.contiguous().view(fmt).float() * ks  # [Hkv, n, D]
        vf = v.contiguous().view(fmt).float() * vs
        q = query[b, 0].float().reshape(kv_heads, groups, dim)  # [Hkv, G, D]
        scores = torch.bmm(q, kf.transpose(1, 2)) * scale  # [Hkv, G, n]
        probs = torch.softmax(scores, dim=-1)
        out[b, 0] = torch.bmm(probs, vf).reshape(q_heads, dim)
    return out
