"""The C ABI's refusals, on the CPU: an entry point whose arguments are valid but for one returns 1, with a message
that names what is wrong, from its own checks and before it reaches a device. Pointers are stand-in addresses (no
check reads through a pointer); each case changes one argument of a call that is otherwise well formed."""

from __future__ import annotations

import math
import re
from pathlib import Path

import pytest
import torch

from economize_amd import _lib

ROOT = Path(__file__).resolve().parents[1]

# (Each case must be refused by the host-side checks: with a device present a call that passed them would launch
# kernels on the stand-in addresses, so the module runs only where there is none.)
pytestmark = pytest.mark.skipif(torch.cuda.is_available(), reason="stand-in addresses: run without a GPU")

FAKE = 1 << 20  # a stand-in address, aligned for every check
BF16, FP8, FP16, FP32 = _lib.ECO_BF16, _lib.ECO_FP8_E4M3, _lib.ECO_FP16, _lib.ECO_FP32


def _names(fn: str) -> list[str]:
    text = (ROOT / "include" / "economize_amd.h").read_text()
    m = re.search(r"\b" + fn + r"\s*\(([^)]*)\)\s*;", text, flags=re.S)
    assert m, fn
    return [re.findall(r"(\w+)\s*$", p.strip())[0] for p in m.group(1).split(",")]


# well-formed calls: every pointer a stand-in unless listed as null (optional inputs), every other argument named
BASE = {
    "eco_paged_decode": dict(
        null=("k_scale", "v_scale", "page_list", "done", "sinks", "mask_bits", "stream"),
        q_format=BF16, sq_b=8, sq_q=8, sq_h=8, kv_format=FP8, num_pages=4, bt_stride=4, bt_cols=4, pl_b=0, pl_h=0,
        n_sel=0, list_page_size=16, so_b=8, so_q=8, so_h=8, batch=1, queries=1, q_heads=8, kv_heads=2,
        head_dim=128, page_size=16, max_seq_len=64, scale=1.0, softcap=0.0, mk_b=0, mk_h=0, mk_q=0, mask_words=0,
        workspace_bytes=1 << 30),
    "eco_kivi_packed_decode": dict(
        null=("mask", "sinks", "stream"),
        q_format=BF16, sq_b=8, sq_h=8, sq_q=8, sk_b=8, sk_h=8, sk_s=8, sv_b=8, sv_h=8, sv_s=8, ring=0, skc_b=32,
        skc_h=32, skc_s=32, sks_b=8, sks_h=8, sks_g=8, svc_b=32, svc_h=32, svc_s=32, svs_b=4, svs_h=4, svs_s=4,
        bits=2, key_group=32, value_group=32, sm_b=0, sm_h=0, sm_q=0, sm_s=0, so_b=8, so_q=8, so_h=8, batch=1,
        queries=1, q_heads=8, kv_heads=2, keys=64, head_dim=128, value_dim=128, scale=1.0, softcap=0.0,
        workspace_bytes=1 << 30),
    "eco_quest_select": dict(
        null=("stream",),
        q_format=BF16, sq_b=8, sq_q=8, sq_h=8, bounds_format=BF16, sb_b=8, sb_h=8, sb_p=8, max_done=4, pages=2,
        first_page=0, batch=1, queries=1, q_heads=8, kv_heads=2, head_dim=128, workspace_bytes=1 << 30),
    "eco_kivi_pack_quantize": dict(
        null=("overflow", "stream"),
        kind=0, format=BF16, ss_b=8, ss_h=8, ss_s=8, src_ring=0, write_back=0, sc_b=32, sc_h=32, sc_s=32, sz_b=8,
        sz_h=8, sz_s=8, batch=1, heads=1, slots=64, head_dim=128, bits=2, group=32, max_tokens=64),
    "eco_kivi_packed_gather": dict(
        null=("stream",),
        kind=0, sc_b=32, sc_h=32, sc_s=32, sz_b=8, sz_h=8, sz_s=8, sr_b=8, sr_h=8, sr_s=8, ring_slots=8, format=BF16,
        so_b=8, so_h=8, so_s=8, batch=1, heads=1, slots=64, head_dim=128, bits=2, group=32),
}

CASES = [
    ("eco_paged_decode", dict(page_size=32), "pages must hold 16 tokens"),
    ("eco_paged_decode", dict(head_dim=96), "head dim must be 64, 128 or 256"),
    ("eco_paged_decode", dict(q_format=FP16, kv_format=BF16), "fp16 queries read an fp8 cache"),
    ("eco_paged_decode", dict(q_format=FP32), "queries must be bf16 or fp16"),
    ("eco_paged_decode", dict(q_heads=7), "not a multiple of the KV heads"),
    ("eco_paged_decode", dict(sq_h=4), "16-byte aligned"),
    ("eco_paged_decode", dict(scale=math.nan), "scale is NaN"),
    ("eco_kivi_packed_decode", dict(bits=3), "bits must be 2, 4 or 8"),
    ("eco_kivi_packed_decode", dict(value_dim=96, value_group=64), "value group must divide"),
    ("eco_kivi_packed_decode", dict(key_codes=FAKE + 1), "codes must be aligned"),
    ("eco_kivi_packed_decode", dict(skc_s=33), "code strides must be multiples"),
    ("eco_kivi_packed_decode", dict(key_scale=FAKE + 2), "key scales and zero points must be aligned"),
    ("eco_kivi_packed_decode", dict(q_format=FP8), "queries must be bf16, fp16 or fp32"),
    ("eco_kivi_packed_decode", dict(keys=0), "need keys > 0"),
    ("eco_kivi_packed_decode", dict(keys_quantized=0), "null quantized counts"),
    ("eco_quest_select", dict(head_dim=12), "multiple of 8 up to 512"),
    ("eco_quest_select", dict(q_heads=6, kv_heads=4), "not a multiple of the KV heads"),
    ("eco_quest_select", dict(kmin=FAKE + 8), "16-byte aligned"),
    ("eco_quest_select", dict(bounds_format=FP8), "bf16, fp16 or fp32"),
    ("eco_kivi_pack_quantize", dict(bits=3), "bits must be 2, 4 or 8"),
    ("eco_kivi_pack_quantize", dict(kind=2), "kind must be 0"),
    ("eco_kivi_pack_quantize", dict(max_tokens=48), "whole groups of tokens"),
    ("eco_kivi_pack_quantize", dict(kind=1, group=48), "value group must divide"),
    ("eco_kivi_pack_quantize", dict(write_back=1, src_ring=8), "ring source is not written back"),
    ("eco_kivi_pack_quantize", dict(head_dim=126), "whole bytes"),
    ("eco_kivi_packed_gather", dict(bits=5), "bits must be 2, 4 or 8"),
    ("eco_kivi_packed_gather", dict(kind=1, group=48), "whole value groups"),
    ("eco_kivi_packed_gather", dict(format=FP8), "bf16, fp16 or fp32"),
    ("eco_kivi_packed_gather", dict(out=0), "null pointer"),
]


def _call(fn: str, bad: dict) -> tuple[int, str]:
    base = dict(BASE[fn])
    null = set(base.pop("null"))
    args = []
    for name, kind in zip(_names(fn), _lib.SIGNATURES[fn][1]):
        if name in bad:
            args.append(bad[name])
        elif name in base:
            args.append(base[name])
        else:
            assert kind is _lib._P, (fn, name)  # every non-pointer argument is named above
            args.append(None if name in null else FAKE)
    lib = _lib.lib()
    rc = getattr(lib, fn)(*args)
    return rc, (lib.eco_last_error() or b"").decode()


@pytest.mark.parametrize("fn,bad,message", CASES, ids=[f"{c[0]}-{'-'.join(c[1])}" for c in CASES])
def test_refused_before_any_device_work(fn: str, bad: dict, message: str) -> None:
    rc, error = _call(fn, bad)
    assert rc == 1, (rc, error)
    assert message in error, error


def test_every_case_names_real_parameters() -> None:
    for fn, bad, _ in CASES:
        names = set(_names(fn))
        assert set(bad) <= names, (fn, set(bad) - names)
        assert set(BASE[fn]) - {"null"} <= names and set(BASE[fn]["null"]) <= names, fn
