"""Pins the torch-CPU restatement of the paged fp8 decode call (oracle/torch_cpu.py, the CPU baseline) against the
numpy oracle: the pages gathered by ``oracle.paged.gather_kv``, decoded by ``oracle.fp8.fp8_decode`` and attended by
``oracle.attention.reference_attention`` (each pinned by its own tests), on ragged rows with GQA and per-head
scales."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import paged as opaged
from oracle.attention import reference_attention
from oracle.torch_cpu import paged_fp8_decode_attention


@pytest.mark.parametrize("fmt,dtype", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_matches_the_numpy_oracle(fmt, dtype) -> None:
    rng = np.random.default_rng(5)
    batch, q_heads, kv_heads, dim = 3, 8, 2, 64
    lens = [100, 1, 333]
    smax = max(lens)
    k = rng.standard_normal((batch, kv_heads, smax, dim)).astype(np.float32)
    v = rng.standard_normal((batch, kv_heads, smax, dim)).astype(np.float32)
    ks = ofp8.head_scales(k, fmt)
    vs = ofp8.head_scales(v, fmt)
    kc = ofp8.fp8_encode(k, fmt, ks.reshape(1, -1, 1, 1))
    vc = ofp8.fp8_encode(v, fmt, vs.reshape(1, -1, 1, 1))
    table, pages = opaged.shuffled_block_table(lens, 16, seed=6)
    kcache, vcache = opaged.scatter_kv(kc, vc, lens, table, pages, 16, 1)
    q = rng.standard_normal((batch, 1, q_heads, dim)).astype(np.float32)
    got = paged_fp8_decode_attention(torch.from_numpy(q), torch.from_numpy(kcache), torch.from_numpy(vcache),
                                     torch.from_numpy(ks), torch.from_numpy(vs), torch.from_numpy(table), lens,
                                     0.125, dtype).numpy()
    gk, gv = opaged.gather_kv(kcache, vcache, table, lens, 16)
    kd = ofp8.fp8_decode(gk, fmt, ks.reshape(1, -1, 1, 1), "f32")
    vd = ofp8.fp8_decode(gv, fmt, vs.reshape(1, -1, 1, 1), "f32")
    mask = (np.arange(smax)[None, :] < np.array(lens)[:, None])[:, None, None, :]
    want = reference_attention(q.transpose(0, 2, 1, 3), kd, vd, mask, 0.125)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)
