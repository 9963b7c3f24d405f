"""Pins the oracle's fp32 attention definition (attention/decode.py:66-103) with brute force and closed forms."""

from __future__ import annotations

import math

import numpy as np

from oracle.attention import reference_attention


def _brute(q, k, v, mask, scale, softcap=None, sinks=None):
    b, hq, nq, _ = q.shape
    hkv, s = k.shape[1], k.shape[2]
    out = np.zeros((b, nq, hq, v.shape[-1]))
    for bi in range(b):
        for h in range(hq):
            kh = h // (hq // hkv)
            for qi in range(nq):
                logits = []
                for t in range(s):
                    if mask is not None and not mask[min(bi, mask.shape[0] - 1), min(h, mask.shape[1] - 1),
                                                     min(qi, mask.shape[2] - 1), t]:
                        continue
                    z = float(np.dot(q[bi, h, qi].astype(np.float64), k[bi, kh, t].astype(np.float64))) * scale
                    if softcap is not None:
                        z = softcap * math.tanh(z / softcap)
                    logits.append((z, t))
                denom = sum(math.exp(z) for z, _ in logits) + (math.exp(sinks[h]) if sinks is not None else 0.0)
                for z, t in logits:
                    out[bi, qi, h] += math.exp(z) / denom * v[bi, kh, t]
    return out


def test_brute_force_gqa_mask_softcap_sinks() -> None:
    rng = np.random.default_rng(0)
    q = rng.standard_normal((2, 6, 3, 8)).astype(np.float32)
    k = rng.standard_normal((2, 2, 11, 8)).astype(np.float32)
    v = rng.standard_normal((2, 2, 11, 5)).astype(np.float32)
    mask = rng.random((2, 6, 3, 11)) > 0.3
    sinks = rng.standard_normal(6).astype(np.float32)
    for kwargs in ({}, {"softcap": 2.0}, {"sinks": sinks}):
        got = reference_attention(q, k, v, mask, 0.35, **kwargs)
        want = _brute(q, k, v, mask, 0.35, kwargs.get("softcap"), kwargs.get("sinks"))
        assert np.allclose(got, want, atol=1e-5, rtol=1e-5)


def test_closed_forms() -> None:
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 4, 2, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 9, 16)).astype(np.float32)
    v = rng.standard_normal((1, 2, 9, 16)).astype(np.float32)
    one = np.zeros((1, 1, 2, 9), bool)
    one[..., 4] = True
    out = reference_attention(q, k, v, one, 0.25)
    assert np.array_equal(out[0, :, 0], np.broadcast_to(v[0, 0, 4], (2, 16)))  # a single visible key
    flat = reference_attention(np.zeros_like(q), k, v, None, 0.25)
    assert np.allclose(flat[0, 0, 0], v[0, 0].mean(0), atol=1e-6)  # uniform scores: the mean
    none = one.copy()
    none[..., 1, :] = False
    assert (reference_attention(q, k, v, none, 0.25)[0, 1] == 0).all()  # a row that sees nothing
    sinks = np.full(4, -np.inf, np.float32)
    assert np.allclose(reference_attention(q, k, v, None, 0.25, sinks=sinks), reference_attention(q, k, v, None, 0.25))


def test_gqa_equals_repeated_heads() -> None:
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 8, 1, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 20, 16)).astype(np.float32)
    v = rng.standard_normal((1, 2, 20, 16)).astype(np.float32)
    a = reference_attention(q, k, v, None, 0.25)
    b = reference_attention(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), None, 0.25)
    assert np.array_equal(a, b)
