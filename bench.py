"""Benchmark of the fp8 paged decode-attention path on one MI355X.

Workload (one "step" = one decode-attention call over the whole batch): Llama-3-8B decode shape, batch 32, one
query per row, 32 query heads over 8 KV heads of 128 channels, K/V in fp8 e4m3 with per-head absmax scales, in
16-token pages assigned from a shuffled page pool. Inputs are resident in HBM before the timed region: q, K and V are
drawn N(0, 1) in bf16 from a seeded generator and quantize-appended into the cache by the fp8 append kernel.

* ``value``: KV-read GB/s at L = 4096 for every row = sum_b L_b * 2 * Hkv * D bytes / seconds per call (split and
  merge kernels together, HIP events on the launch stream around ``--steps`` calls after ``--warmup`` calls).
* ``roofline``: the call is one kernel launch (``paged_attention_kernel``): algorithmic bytes per launch (KV + q +
  out + block table + lengths + scales) over its average launch time, against 8 TB/s.
* ``ragged``: the same with lengths drawn uniformly from [1024, 8192] (mean 4608).
* ``paths``: the other decode configurations (KIVI decode and verification, Quest, the dense, gathered, vLLM-cells
  and KIVI packed paths, the captured Quest step), each with its algorithmic bytes, timed over at least 200 calls
  after at least 20 warm-up calls and 50 ms of them.
* ``cpu_baseline``: the torch-CPU fp32 restatement of the call (oracle/torch_cpu.py) over whole calls of the
  L = 4096 workload on the host's share of cores (1 warmup, median of 5), with the core count and CPU model; its
  output is also the check of the timed GPU call's output.

Every path's timed calls rotate over distinct copies of the cache (1 + ceil(384 MB / bytes per call) copies of the
K/V data, KIVI pages and rings, Quest bounds), the way a decode step reads a different layer's cache at every call
while the layers share the block table, the lengths and, here, the query: so no call finds its cache data in the
256 MB Infinity Cache from its previous use (with a single copy the L = 4096 call reads about a sixth of its bytes
from that cache). ``--single-copy`` measures the single-copy figures.

``--length-sweep`` prints, instead of the line above, per-call times against the context length at a fixed batch
(the fp8 shape at B = 32, the KIVI int2 / int4 decode at B = 16) and the least-squares line over L >= 4096, whose
intercept is the per-call time that does not grow with the context.

``--gpus`` must be 1: the path runs on one GPU.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BATCH, Q_HEADS, KV_HEADS, HEAD_DIM, PAGE = 32, 32, 8, 128, 16
TRAFFIC_FILE = ROOT / "profiles" / "paged_decode_fp8_b32_l4096_traffic.txt"


def build_workload(lens: list[int], seed: int):
    """q [B, 1, Hq, D] bf16, a fp8 e4m3 paged cache holding every row's lens[b] tokens, block table, lengths."""
    import numpy as np
    import torch

    from economize_amd.paged import PagedKVCache, head_scales, paged_append

    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(seed)
    smax = max(lens)
    q = torch.randn(BATCH, 1, Q_HEADS, HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    need = [-(-n // PAGE) for n in lens]
    total = sum(need) + 3
    order = np.random.default_rng(seed + 1).permutation(total)
    table = np.full((BATCH, max(need)), -1, dtype=np.int32)
    at = 0
    for b, n in enumerate(need):
        table[b, :n] = order[at: at + n]
        at += n
    block_table = torch.from_numpy(table).to(device)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=device)
    k = torch.randn(BATCH, KV_HEADS, smax, HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(BATCH, KV_HEADS, smax, HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    valid = (torch.arange(smax, device=device)[None, :] < seq_lens[:, None])[:, None, :, None]
    k = torch.where(valid, k, 0)
    v = torch.where(valid, v, 0)
    cache = PagedKVCache.empty(total, KV_HEADS, HEAD_DIM, torch.float8_e4m3fn, device,
                               head_scales(k), head_scales(v))
    for b, n in enumerate(lens):
        t = torch.arange(n, device=device)
        slots = (block_table[b, t // PAGE] * PAGE + t % PAGE).to(torch.int32)
        paged_append(cache, k[b, :, :n].transpose(0, 1), v[b, :, :n].transpose(0, 1), slots)
    torch.cuda.synchronize()
    del k, v
    return q, cache, block_table, seq_lens


MIN_WARMUP_S = 0.0  # seconds of warm-up calls at least, besides their count (set for the path rows)


def time_calls(fn, steps: int, warmup: int) -> float:
    """Average seconds per call of ``fn`` over ``steps`` calls after ``warmup`` calls, and after at least
    MIN_WARMUP_S seconds of them (HIP events on the current stream, which is the stream the kernels launch on)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start_warm = time.perf_counter()
    while time.perf_counter() - start_warm < MIN_WARMUP_S:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / steps


def kv_bytes(lens: list[int]) -> int:
    return sum(lens) * 2 * KV_HEADS * HEAD_DIM  # one byte per fp8 element, K and V


def call_bytes(lens: list[int]) -> int:
    """Algorithmic bytes of one call: K/V, the query and the output (bf16), the block table entries, the lengths and
    the scales."""
    pages = sum(-(-n // PAGE) for n in lens)
    return kv_bytes(lens) + 2 * BATCH * Q_HEADS * HEAD_DIM * 2 + pages * 4 + BATCH * 4 + 2 * KV_HEADS * 4


INFINITY_CACHE_MARGIN = 384e6  # bytes the other copies must hold, beyond the 256 MB Infinity Cache
SINGLE_COPY = False  # --single-copy: every call on the same inputs


def copies_for(nbytes: int) -> int:
    """Distinct input copies the timed calls rotate over, so that a call's data has left the Infinity Cache."""
    return 1 if SINGLE_COPY else 1 + math.ceil(INFINITY_CACHE_MARGIN / nbytes)


def rotating(calls: list):
    """One function that runs calls[0], calls[1], ... in turn."""
    state = [0]

    def call() -> None:
        calls[state[0] % len(calls)]()
        state[0] += 1

    return call


def measure(lens: list[int], steps: int, warmup: int, seed: int) -> dict:
    import torch

    from economize_amd.paged import new_workspace, paged_decode_attention, workspace_size

    smax = max(lens)
    q, cache, table, seq_lens = build_workload(lens, seed)
    caches = [cache] + [dataclasses.replace(cache, keys=cache.keys.clone(), values=cache.values.clone())
                        for _ in range(1, copies_for(call_bytes(lens)))]
    out = torch.empty_like(q)
    ws = new_workspace(workspace_size(BATCH, 1, Q_HEADS, KV_HEADS, HEAD_DIM, smax, 0, cache.dtype), q.device)

    def call_on(c):
        return lambda: paged_decode_attention(q, c, table, seq_lens, smax, out=out, workspace=ws)

    seconds = time_calls(rotating([call_on(c) for c in caches]), steps, warmup)
    return {
        "seconds": seconds,
        "kv_bytes": kv_bytes(lens),
        "call_bytes": call_bytes(lens),
        "copies": len(caches),
        "workload": (q, cache, table, seq_lens, out),
    }


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(workload, lens: list[int], reps: int = 5) -> dict:
    """The torch-CPU fp32 restatement of the call (oracle/torch_cpu.py: page gather, exact fp8 decode times the head
    scale, fp32 attention) over the whole batch, on the host's share of cores (OMP_NUM_THREADS, else every core):
    one warmup call, then the median of ``reps`` whole calls. Its output is the check of the timed GPU call's output
    (atol 2e-3 / rtol 1e-2 against this fp32 definition)."""
    import statistics

    import torch

    from oracle.torch_cpu import paged_fp8_decode_attention

    q, cache, table, _, out = workload
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    args = (q.cpu(), cache.keys.view(torch.uint8).cpu(), cache.values.view(torch.uint8).cpu(), cache.k_scale.cpu(),
            cache.v_scale.cpu(), table.cpu(), lens, 1.0 / math.sqrt(HEAD_DIM))
    want = paged_fp8_decode_attention(*args)  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        paged_fp8_decode_attention(*args)
        times.append(time.perf_counter() - t0)
    per_call = statistics.median(times)
    got = out.float().cpu()
    err = (got - want).abs()
    within = bool((err <= 2e-3 + 1e-2 * want.abs()).all())
    return {
        "value": round(kv_bytes(lens) / per_call / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu": cpu_model(),
        "us_per_call": round(per_call * 1e6, 1),
        "sample": f"whole calls of the timed L=4096 workload ({BATCH} rows): 1 warmup + median of {reps}, torch-CPU "
                  f"fp32 (page gather, fp8 decode, attention) on {threads} threads",
        "gpu_output_check": {"max_abs_err": round(float(err.max()), 6), "within_atol_2e-3_rtol_1e-2": within},
    }


# ---- the other paths: KIVI decode, Quest selection + gathered attention, KIVI verification (MFMA) -------------------


def _shuffled_table(batch: int, pages_per_row: list[int], seed: int, device):
    import numpy as np
    import torch

    total = sum(pages_per_row) + 3
    order = np.random.default_rng(seed).permutation(total)
    table = np.full((batch, max(pages_per_row)), -1, dtype=np.int32)
    at = 0
    for b, n in enumerate(pages_per_row):
        table[b, :n] = order[at: at + n]
        at += n
    return torch.from_numpy(table).to(device), total


def kivi_workload(batch, queries, q_heads, kv_heads, lens, bits, seed, residual=128, headroom=256):
    """A KIVI cache holding every row's lens[b] tokens (committed: lens[b] - queries), filled by the GPU kernels:
    K/V/q N(0, 1) in bf16 with 4 of 128 key channels scaled by 10, 32-token pages in a shuffled pool."""
    import torch

    from economize_amd.kivi import PagedKIVICache, kivi_append, kivi_quantize

    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(seed)
    smax = max(lens)
    q = torch.randn(batch, queries, q_heads, HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(batch, kv_heads, smax, HEAD_DIM, generator=gen, device=device)
    k[..., torch.randperm(HEAD_DIM, generator=gen, device=device)[:4]] *= 10.0
    k = k.to(torch.bfloat16)
    v = torch.randn(batch, kv_heads, smax, HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    table, pages = _shuffled_table(batch, [-(-n // 32) for n in lens], seed + 1, device)
    cache = PagedKIVICache.empty(pages, batch, kv_heads, HEAD_DIM, bits, device, residual=residual,
                                 headroom=headroom)
    committed = torch.tensor([n - queries for n in lens], dtype=torch.int32, device=device)
    kq = (committed // residual) * residual
    vq = torch.clamp(committed - residual, min=0)
    zeros = torch.zeros(batch, dtype=torch.int32, device=device)
    kivi_quantize(cache, table, k, "k", zeros, kq.to(torch.int32), smax)
    kivi_quantize(cache, table, v, "v", zeros, vq.to(torch.int32), smax)
    ring = cache.ring
    rows = torch.cat([torch.full((min(n, ring),), b, dtype=torch.int32) for b, n in enumerate(lens)]).to(device)
    pos = torch.cat([torch.arange(max(0, n - ring), n, dtype=torch.int32) for n in lens]).to(device)
    kivi_append(cache, k[rows.long(), :, pos.long()], v[rows.long(), :, pos.long()], rows, pos)
    cache.keys_quantized.copy_(kq)
    cache.values_quantized.copy_(vq)
    torch.cuda.synchronize()
    del k, v
    return q, cache, table, torch.tensor(lens, dtype=torch.int32, device=device), kq.tolist(), vq.tolist()


def kivi_call_bytes(lens, kq, vq, bits, batch, queries, q_heads, kv_heads) -> int:
    """Algorithmic bytes of a KIVI call: per (row, KV head) the codes and fp16 scales / zero points of the quantized
    keys and values (D * bits / 8 + 4 D / 32 bytes per token each) and the bf16 ring entries of the rest (the
    reference's kivi_bytes, techniques/kv_quant/kivi.py:163-175), plus q, out, table entries and counts."""
    d = HEAD_DIM
    per_q = d * bits // 8 + 4 * d // 32
    kv = sum(kv_heads * (k * per_q + v * per_q + (2 * n - k - v) * d * 2) for n, k, v in zip(lens, kq, vq))
    return kv + 2 * batch * queries * q_heads * d * 2 + sum(-(-n // 32) for n in lens) * 4 + 3 * batch * 4


def measure_kivi(bits: int, steps: int, warmup: int, seed: int, batch=16, queries=1, q_heads=32, kv_heads=8,
                 lens=None) -> dict:
    import torch

    from economize_amd.kivi import kivi_decode_attention

    lens = lens or [8192] * batch
    q, cache, table, seq, kq, vq = kivi_workload(batch, queries, q_heads, kv_heads, lens, bits, seed)
    nbytes = kivi_call_bytes(lens, kq, vq, bits, batch, queries, q_heads, kv_heads)
    caches = [cache] + [dataclasses.replace(cache, blocks=cache.blocks.clone(), k_ring=cache.k_ring.clone(),
                                            v_ring=cache.v_ring.clone()) for _ in range(1, copies_for(nbytes))]
    out = torch.empty_like(q)
    smax = max(lens)

    def call_on(c):
        return lambda: kivi_decode_attention(q, c, table, seq, smax, out=out)

    seconds = time_calls(rotating([call_on(c) for c in caches]), steps, warmup)
    flops = sum(2 * 2 * kv_heads * (q_heads // kv_heads) * queries * n * HEAD_DIM for n in lens)
    copies = len(caches)
    del caches, cache
    return {"us_per_call": round(seconds * 1e6, 2), "algorithmic_bytes": nbytes,
            "gb_s": round(nbytes / seconds / 1e9, 1), "hbm_frac": round(nbytes / seconds / 1e9 / HBM_PEAK_GBS, 4),
            "tflop_s": round(flops / seconds / 1e12, 2), "copies": copies}


def quest_workload(seed: int, batch: int, q_heads: int, kv_heads: int, length: int, budget: int, planted: int):
    """bf16 K/V in 16-token pages; per (row, KV head) `planted` pages whose keys are the group's first query plus
    0.1 N(0, 1); the bounds of the committed pages (the cache maintains them). Returns the query [B, Hq, 1, D], the
    cache, the block table, the lengths and the QuestPages."""
    import torch

    from economize_amd.paged import PagedKVCache, paged_append
    from economize_amd.quest import QuestPages, paged_page_bounds

    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(batch, 1, q_heads, HEAD_DIM, generator=gen, device=device).to(torch.bfloat16)
    pages_per_row = length // PAGE
    table, total = _shuffled_table(batch, [pages_per_row] * batch, seed + 1, device)
    cache = PagedKVCache.empty(total, kv_heads, HEAD_DIM, torch.bfloat16, device)
    groups = q_heads // kv_heads
    for b in range(batch):
        k = torch.randn(length, kv_heads, HEAD_DIM, generator=gen, device=device)
        v = torch.randn(length, kv_heads, HEAD_DIM, generator=gen, device=device)
        for h in range(kv_heads):
            chosen = torch.randperm(pages_per_row - 1, generator=gen, device=device)[:planted]
            idx = (chosen[:, None] * PAGE + torch.arange(PAGE, device=device)[None, :]).reshape(-1)
            k[idx, h] = q[b, 0, h * groups].float() + 0.1 * torch.randn(idx.numel(), HEAD_DIM, generator=gen,
                                                                           device=device)
        t = torch.arange(length, device=device)
        slots = (table[b, t // PAGE] * PAGE + t % PAGE).to(torch.int32)
        paged_append(cache, k.to(torch.bfloat16), v.to(torch.bfloat16), slots)
    done = (length - 1) // PAGE
    kmin, kmax = paged_page_bounds(cache, table, 0, done, PAGE)
    pages = budget // PAGE - 1
    qp = QuestPages(kmin, kmax, torch.full((batch,), done, dtype=torch.int32, device=device), done, done, PAGE, pages)
    seq = torch.full((batch,), length, dtype=torch.int32, device=device)
    return q.transpose(1, 2), cache, table, seq, qp


def measure_quest(steps: int, warmup: int, seed: int, batch=8, q_heads=32, kv_heads=8, length=32768, budget=1024,
                  planted=32) -> dict:
    """Quest decode: a call is the selection (scores + top-k) plus the attention over the selected pages and the
    dense tail, over the workload of quest_workload."""
    import torch

    from economize_amd.quest import paged_quest_decode_attention

    d = HEAD_DIM
    done = (length - 1) // PAGE
    pages = budget // PAGE - 1
    tail = length - done * PAGE
    nbytes = (batch * kv_heads * (2 * d * 2 * done + (pages * PAGE + tail) * 2 * d * 2 + done * 4 * 2)
              + 2 * batch * q_heads * d * 2 + batch * kv_heads * pages * 4 * 2)
    query, cache, table, seq, qp = quest_workload(seed, batch, q_heads, kv_heads, length, budget, planted)
    loads = [(cache, qp)] + [(dataclasses.replace(cache, keys=cache.keys.clone(), values=cache.values.clone()),
                              dataclasses.replace(qp, kmin=qp.kmin.clone(), kmax=qp.kmax.clone()))
                             for _ in range(1, copies_for(nbytes))]
    out = torch.empty(batch, 1, q_heads, d, dtype=torch.bfloat16, device="cuda:0")

    def call_on(load):
        c, pages_ = load
        return lambda: paged_quest_decode_attention(query, c, table, seq, length, pages_, out=out)

    seconds = time_calls(rotating([call_on(load) for load in loads]), steps, warmup)
    torch.cuda.synchronize()
    copies = len(loads)
    del loads, cache, qp
    return {"us_per_call": round(seconds * 1e6, 2), "algorithmic_bytes": nbytes,
            "gb_s": round(nbytes / seconds / 1e9, 1), "hbm_frac": round(nbytes / seconds / 1e9 / HBM_PEAK_GBS, 4),
            "dense_bytes_avoided": batch * kv_heads * length * 2 * d * 2, "copies": copies}


def _result(seconds: float, nbytes: int, copies: int, **extra) -> dict:
    return {"us_per_call": round(seconds * 1e6, 2), "algorithmic_bytes": int(nbytes),
            "gb_s": round(nbytes / seconds / 1e9, 1), "hbm_frac": round(nbytes / seconds / 1e9 / HBM_PEAK_GBS, 4),
            "copies": copies, **extra}


def measure_dense(steps: int, warmup: int, seed: int, kv_dtype, batch=32, q_heads=32, kv_heads=8, length=4096) -> dict:
    """decode_attention over dense [B, Hkv, L, D] buffers (a model cache's own layout; fp8 views: the fused fp8 cache's
    dense buffers): K and V read once, plus the query and output."""
    import torch

    from economize_amd.decode import decode_attention

    d = HEAD_DIM
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    es = torch.empty((), dtype=kv_dtype).element_size()
    nbytes = batch * kv_heads * length * 2 * d * es + 2 * batch * q_heads * d * 2
    q = torch.randn(batch, 1, q_heads, d, generator=gen, device="cuda:0").to(torch.bfloat16).transpose(1, 2)
    copies = copies_for(nbytes)
    loads = []
    for _ in range(copies):
        k = torch.randn(batch, kv_heads, length, d, generator=gen, device="cuda:0").to(kv_dtype)
        v = torch.randn(batch, kv_heads, length, d, generator=gen, device="cuda:0").to(kv_dtype)
        loads.append((k, v))
    out = torch.empty(batch, 1, q_heads, d, dtype=torch.bfloat16, device="cuda:0")
    scale = 1 / math.sqrt(d)
    seconds = time_calls(rotating([lambda k=k, v=v: decode_attention(q, k, v, None, scale, out=out)
                                   for k, v in loads]), steps, warmup)
    del loads
    return _result(seconds, nbytes, copies)


def measure_gathered(steps: int, warmup: int, seed: int, batch=32, q_heads=32, kv_heads=8, prompt=3968, tail=128,
                     keep=0.5) -> dict:
    """gathered_decode_attention: every (row, KV head) keeps a random half of its prompt entries (an eviction's
    compacted entries) and reads them plus a dense tail of generated tokens; bytes are the entries read."""
    import numpy as np
    import torch

    from economize_amd.gathered import GatheredKV, gathered_decode_attention

    d = HEAD_DIM
    slots = prompt + tail
    rng = np.random.default_rng(seed)
    cap = int(prompt * keep)
    count = torch.full((batch, kv_heads), cap, dtype=torch.int32, device="cuda:0")
    index = torch.from_numpy(np.sort(np.stack([rng.choice(prompt, cap, replace=False)
                                               for _ in range(batch * kv_heads)]), axis=1).astype(np.int32)) \
        .view(batch, kv_heads, cap).cuda()
    start = torch.full((batch,), prompt, dtype=torch.int32, device="cuda:0")
    nbytes = batch * kv_heads * (cap + tail) * 2 * d * 2 + 2 * batch * q_heads * d * 2 + index.numel() * 4
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    q = torch.randn(batch, 1, q_heads, d, generator=gen, device="cuda:0").to(torch.bfloat16).transpose(1, 2)
    copies = copies_for(nbytes)
    loads = []
    for _ in range(copies):
        k = torch.randn(batch, kv_heads, slots, d, generator=gen, device="cuda:0").to(torch.bfloat16)
        v = torch.randn(batch, kv_heads, slots, d, generator=gen, device="cuda:0").to(torch.bfloat16)
        ck = torch.randn(batch, kv_heads, cap, d, generator=gen, device="cuda:0").to(torch.bfloat16)
        cv = torch.randn(batch, kv_heads, cap, d, generator=gen, device="cuda:0").to(torch.bfloat16)
        loads.append((k, v, GatheredKV(ck, cv, index, count, start, prompt - cap)))
    out = torch.empty(batch, 1, q_heads, d, dtype=torch.bfloat16, device="cuda:0")
    scale = 1 / math.sqrt(d)
    seconds = time_calls(rotating([lambda k=k, v=v, g=g: gathered_decode_attention(q, k, v, None, scale, g, out=out)
                                   for k, v, g in loads]), steps, warmup)
    del loads
    return _result(seconds, nbytes, copies, dense_bytes=batch * kv_heads * slots * 2 * d * 2)


def measure_cells(steps: int, warmup: int, seed: int, batch=16, q_heads=32, kv_heads=8, length=8192, bits=2,
                  page=32, residual=128) -> dict:
    """paged_kivi_attention over vLLM's KIVI cells (bf16 entries, groups of 32), one query per request, after
    quantize_committed at this step's schedule (residual 128): keys below ((L - 1) / R) R and values below L - 1 - R
    are read through their codes, scales and flags as the reference's kernel reads them, the rest from their dense
    entries. Algorithmic bytes: per (request, KV head) kq (D bits / 8 + 2 (2 D) / G + 1) + vq (D bits / 8 + 4 D / vg +
    1) + (2 L - kq - vq) 2 D, plus queries, outputs and the block table."""
    import torch

    from economize_amd.vllm_kivi import cell_layout, paged_kivi_attention, quantize_committed

    d, group = HEAD_DIM, 32
    layout = cell_layout(d, torch.bfloat16, bits, group)
    per_row = length // page
    pages = batch * per_row
    c = length - 1  # tokens committed before the step
    kq, vq = (c // residual) * residual, max(0, c - residual)
    per_head = (kq * (d * bits // 8 + 2 * 2 * d // group + 1) + vq * (d * bits // 8 + 2 * 2 * (d // group) + 1)
                + (2 * length - kq - vq) * 2 * d)
    nbytes = batch * kv_heads * per_head + 2 * batch * q_heads * d * 2 + pages * 4
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    table = torch.randperm(pages, generator=gen, device="cuda:0").view(batch, per_row).to(torch.int32)
    q = torch.randn(batch, q_heads, d, generator=gen, device="cuda:0").to(torch.bfloat16)
    qsl = torch.arange(batch + 1, dtype=torch.int32, device="cuda:0")
    seq = torch.full((batch,), length, dtype=torch.int32, device="cuda:0")
    copies = copies_for(nbytes)
    caches = []
    for _ in range(copies):
        cache = torch.randn(pages, kv_heads, page, layout.size // 2, generator=gen, device="cuda:0").to(torch.bfloat16)
        cache.view(torch.uint8)[..., layout.off_flag: layout.off_flag + 2] = 0  # every cell full precision
        quantize_committed(cache, layout, residual, table, qsl, seq, torch.zeros(batch, dtype=torch.int32,
                                                                                 device="cuda:0"))
        caches.append(cache)
    out = torch.empty_like(q)
    seconds = time_calls(rotating([lambda c=c: paged_kivi_attention(q, c, layout, table, qsl, seq, 1, length, out=out)
                                   for c in caches]), steps, warmup)
    cell_bytes = pages * kv_heads * page * layout.size
    del caches
    return _result(seconds, nbytes, copies, cache_bytes=cell_bytes)


def measure_quest_graph(steps: int, warmup: int, seed: int, batch=8, q_heads=32, kv_heads=8, length=32768,
                        budget=1024) -> dict:
    """A Quest decode step with its metadata on the device (QuestState): one appended token per row with the bounds
    refresh in the same launch (eco_paged_append_quest), the selection with a static max_done and the page-list
    attention, captured once in a HIP graph and replayed, against the same step launched eagerly."""
    import torch

    from economize_amd.quest import QuestState, paged_quest_decode_attention

    d = HEAD_DIM
    query, cache, table, seq, qp = quest_workload(seed, batch, q_heads, kv_heads, length, budget, 32)
    pages = budget // PAGE - 1
    state = QuestState(batch, kv_heads, d, length // PAGE, PAGE, pages, "cuda:0")  # the table's capacity
    committed = (seq - 1).contiguous()
    state.refresh(cache, table, committed)
    k_new = torch.zeros(batch, kv_heads, d, dtype=torch.bfloat16, device="cuda:0")
    slots = (table[:, -1] * PAGE + PAGE - 1).contiguous()  # each step rewrites every row's last token
    out = torch.empty(batch, 1, q_heads, d, dtype=torch.bfloat16, device="cuda:0")
    handle = state.pages_handle()

    def step() -> None:
        state.append(cache, k_new, k_new, slots, table, committed)
        paged_quest_decode_attention(query, cache, table, seq, length, handle, out=out)  # static: the capacity

    eager = time_calls(step, steps, warmup)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    replay = time_calls(graph.replay, steps, warmup)
    done = (length - 1) // PAGE
    tail = length - done * PAGE
    nbytes = (batch * kv_heads * (2 * d * 2 * state.max_pages + (pages * PAGE + tail) * 2 * d * 2)
              + 2 * batch * q_heads * d * 2)
    del graph, cache, state
    return {"us_per_step_graph": round(replay * 1e6, 2), "us_per_step_eager": round(eager * 1e6, 2),
            "algorithmic_bytes": int(nbytes), "gb_s_graph": round(nbytes / replay / 1e9, 1),
            "hbm_frac_graph": round(nbytes / replay / 1e9 / HBM_PEAK_GBS, 4), "copies": 1}


def measure_kivi_packed(steps: int, warmup: int, seed: int, bits: int = 8, group: int = 128, batch=16, q_heads=32,
                        kv_heads=8, length=8192, residual=128) -> dict:
    """kivi_decode_attention over the reference's KIVIPacked layout (dense buffers beside the codes, the fused
    cache): every row quantized up to length - residual (keys in whole groups), the rest read from the buffers; bytes
    are the codes, scales and zero points of the quantized slots plus the full-precision rest."""
    import torch

    from economize_amd.kivi_packed import KIVIPackedStore, kivi_decode_attention

    d = HEAD_DIM
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    kq = (length - residual) // group * group
    vq = length - residual
    per_token = d * bits / 8
    nbytes = int(batch * kv_heads * (kq * per_token + kq // group * d * 4 + vq * per_token + vq * 4 +
                                     (length - kq + length - vq) * d * 2) + 2 * batch * q_heads * d * 2)
    q = torch.randn(batch, 1, q_heads, d, generator=gen, device="cuda:0").to(torch.bfloat16).transpose(1, 2)
    copies = copies_for(nbytes)
    loads = []
    for _ in range(copies):
        k = torch.randn(batch, kv_heads, length, d, generator=gen, device="cuda:0").to(torch.bfloat16)
        v = torch.randn(batch, kv_heads, length, d, generator=gen, device="cuda:0").to(torch.bfloat16)
        store = KIVIPackedStore(batch, kv_heads, length, d, d, bits, group, "cuda:0")
        rows = lambda x: torch.full((batch,), x, dtype=torch.int32, device="cuda:0")  # noqa: E731
        store.quantize(k, "k", rows(0), rows(kq), kq, write_back=True)
        store.quantize(v, "v", rows(0), rows(vq), vq, write_back=True)
        store.keys_quantized.fill_(kq)
        store.values_quantized.fill_(vq)
        loads.append((k, v, store.record(length)))
    out = torch.empty(batch, 1, q_heads, d, dtype=torch.bfloat16, device="cuda:0")
    scale = 1 / math.sqrt(d)
    seconds = time_calls(rotating([lambda k=k, v=v, r=r: kivi_decode_attention(q, k, v, None, scale, r, out=out)
                                   for k, v, r in loads]), steps, warmup)
    del loads
    return _result(seconds, nbytes, copies)


PATH_STEPS = 200
PATH_WARMUP = 20
PATH_WARMUP_S = 0.05


def measure_next_rows(steps: int, warmup: int, seed: int) -> dict:
    import torch

    rows = {}
    for name, workload, fn in (
        ("dense_decode_bf16", "decode_attention over dense bf16 [B, Hkv, L, D] buffers, B=32 Hq=32 Hkv=8 D=128 L=4096",
         lambda: measure_dense(steps, warmup, seed, torch.bfloat16)),
        ("dense_decode_fp8", "decode_attention over dense fp8 e4m3 views (the fused fp8 cache), same shape",
         lambda: measure_dense(steps, warmup, seed, torch.float8_e4m3fn)),
        ("gathered_decode", "gathered_decode_attention, B=32 Hq=32 Hkv=8 D=128, half of a 3968-token prompt kept per "
                            "KV head + 128 tail tokens, bf16", lambda: measure_gathered(steps, warmup, seed)),
        ("kivi_cells_attention", "paged_kivi_attention over vLLM KIVI cells (bf16 entries, int2, G=32, R=128, "
                                 "quantized by quantize_committed), B=16 Hq=32 Hkv=8 D=128 L=8192, one query per "
                                 "request",
         lambda: measure_cells(steps, warmup, seed)),
        ("kivi_packed_int8_g128", "kivi_decode_attention over the reference's KIVIPacked layout (8-bit codes, groups "
                                  "of 128, beside bf16 buffers: a configuration the paged KIVI cache does not hold), "
                                  "B=16 Hq=32 Hkv=8 D=128 L=8192, R=128",
         lambda: measure_kivi_packed(steps, warmup, seed)),
        ("quest_graph_step", "Quest decode step with device metadata (append with the bounds refresh in one launch "
                             "+ selection + attention), B=8 Hq=32 Hkv=8 D=128 L=32768, captured graph vs eager",
         lambda: measure_quest_graph(steps, warmup, seed)),
    ):
        rows[name] = {"workload": workload, **fn()}
        report_path(name, rows[name])
        torch.cuda.empty_cache()
    return rows


def report_path(name: str, row: dict) -> None:
    """One line on stderr per measured path (the JSON line on stdout carries the figures)."""
    us = row.get("us_per_call", row.get("us_per_step_graph"))
    print(f"path {name}: {us} us", file=sys.stderr, flush=True)


def measure_paths(steps: int, warmup: int, seed: int) -> dict:
    """The other configurations' rows, each timed over at least PATH_STEPS calls after at least PATH_WARMUP warm-up
    calls and PATH_WARMUP_S seconds of them, whatever --steps / --warmup say (the headline keeps exactly those): the
    first KIVI calls of a process read slower until the GPU has run them for a while (B=16 L=8192 int2: 52.2-52.5 us
    over 200 calls after 20, 47.7 us after 1000, about 50 ms, in a fresh process; about 48 us later in the process
    on fresh inputs after 20), while a decode loop calls its kernels back to back."""
    global MIN_WARMUP_S
    MIN_WARMUP_S = PATH_WARMUP_S
    try:
        return _measure_paths(max(steps, PATH_STEPS), max(warmup, PATH_WARMUP), seed)
    finally:
        MIN_WARMUP_S = 0.0


def _measure_paths(steps: int, warmup: int, seed: int) -> dict:
    import numpy as np
    import torch

    paths = {"kivi_int2_decode": {"workload": "KIVI int2 decode, B=16 Hq=32 Hkv=8 D=128 L=8192, G=32 R=128",
                                  **measure_kivi(2, steps, warmup, seed)}}
    report_path("kivi_int2_decode", paths["kivi_int2_decode"])
    paths["kivi_int4_decode"] = {"workload": "KIVI int4 decode, B=16 Hq=32 Hkv=8 D=128 L=8192, G=32 R=128",
                                 **measure_kivi(4, steps, warmup, seed)}
    report_path("kivi_int4_decode", paths["kivi_int4_decode"])
    torch.cuda.empty_cache()
    paths["quest_decode"] = {"workload": "Quest decode, B=8 Hq=32 Hkv=8 D=128 L=32768 bf16, 63 pages + tail",
                             **measure_quest(steps, warmup, seed)}
    report_path("quest_decode", paths["quest_decode"])
    torch.cuda.empty_cache()
    lens = np.random.default_rng(seed + 200).integers(1024, 4097, 64).tolist()
    paths["kivi_int4_verify"] = {
        "workload": "KIVI int4 speculative verification, B=64 Q=8 Hq=64 Hkv=8 D=128 L~U[1024,4096], causal draft",
        "sum_len": int(sum(lens)),
        **measure_kivi(4, steps, warmup, seed, batch=64, queries=8, q_heads=64, kv_heads=8, lens=lens)}
    report_path("kivi_int4_verify", paths["kivi_int4_verify"])
    torch.cuda.empty_cache()
    paths.update(measure_next_rows(steps, warmup, seed))
    return paths


def fit_line(xs: list[float], ys: list[float]) -> tuple[float, float]:
    """Least-squares slope and intercept of ys against xs."""
    n = len(xs)
    mx, my = sum(xs) / n, sum(ys) / n
    sxx = sum((x - mx) ** 2 for x in xs)
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sxx
    return slope, my - slope * mx


def measure_length_sweep(steps: int, warmup: int, seed: int) -> dict:
    """Per-call time against the context length, every row of a batch at the same length: the fp8 decode at B=32
    (lengths 2048 .. 16384) and the KIVI int2 / int4 decode at B=16 (2048 .. 16384), each timed as its bench row is
    (rotating copies; from these lengths up a call's kernel outlasts its host-side launch). The least-squares line
    through the lengths from 4096 up gives the microseconds per 1024 tokens of every row and the intercept: the time
    of a call that does not grow with the context (the launch, the first dependent loads, the uneven ends of the
    waves' ranges and the merges)."""
    import torch

    def family(name, lengths, fit_from, time_us):
        times = []
        for n in lengths:
            times.append(round(time_us(n), 2))
            print(f"length sweep: {name} L={n}: {times[-1]} us per call", file=sys.stderr, flush=True)
            torch.cuda.empty_cache()
        xs = [n / 1024 for n in lengths if n >= fit_from]
        slope, intercept = fit_line(xs, [t for n, t in zip(lengths, times) if n >= fit_from])
        return {"lengths": list(lengths), "us_per_call": times,
                "fit": {"lengths": [n for n in lengths if n >= fit_from], "us_per_1024_tokens": round(slope, 3),
                        "intercept_us": round(intercept, 2)}}

    def paged_us(n):
        r = measure([n] * BATCH, steps, warmup, seed)
        return r["seconds"] * 1e6

    sweep = {"paged_fp8_b32": family("paged_fp8_b32", (2048, 4096, 8192, 16384), 4096, paged_us)}
    for bits in (2, 4):
        sweep[f"kivi_int{bits}_b16"] = family(
            f"kivi_int{bits}_b16", (2048, 4096, 8192, 16384), 4096,
            lambda n, bits=bits: measure_kivi(bits, steps, warmup, seed, batch=16, lens=[n] * 16)["us_per_call"])
    return sweep


def traffic_per_launch() -> float | None:
    """HBM bytes per split-kernel launch from the committed rocprofv3 counter summary, if present."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--fixed-only", action="store_true", help="skip the ragged-length run (for profiling)")
    parser.add_argument("--no-paths", action="store_true", help="skip the KIVI and Quest measurements")
    parser.add_argument("--single-copy", action="store_true",
                        help="time every call on the same inputs (partly served by the 256 MB Infinity Cache)")
    parser.add_argument("--length-sweep", action="store_true",
                        help="only print per-call times against the context length (fp8 B=32, KIVI int2/int4 B=16)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run a plain device copy of 256 MiB, 20 times (the reference kernel for scaling the "
                             "FETCH_SIZE / WRITE_SIZE counters of rocprofv3)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the decode-attention path shards by (batch row, KV head) with no "
              f"collective, so --gpus {args.gpus} is not run; use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    global SINGLE_COPY
    SINGLE_COPY = args.single_copy
    if args.copy_calibration:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_launch": src.numel(), "launches": 20}), flush=True)
        return

    if args.length_sweep:
        print(json.dumps({"length_sweep": measure_length_sweep(args.steps, args.warmup, args.seed)}), flush=True)
        return

    fixed = [4096] * BATCH
    head = measure(fixed, args.steps, args.warmup, args.seed)
    print(f"headline: {head['seconds'] * 1e6:.2f} us", file=sys.stderr, flush=True)
    ragged_lens = np.random.default_rng(args.seed + 100).integers(1024, 8193, BATCH).tolist()
    ragged = None if args.fixed_only else measure(ragged_lens, args.steps, args.warmup, args.seed + 1)
    if ragged is not None:
        print(f"ragged: {ragged['seconds'] * 1e6:.2f} us", file=sys.stderr, flush=True)
    # the paths before the CPU baseline: its 10-30 s leave the GPU idle, and a call timed right after an idle GPU
    # reads slower (the first KIVI path: about 3 us)
    paths = None if (args.no_paths or args.fixed_only) else measure_paths(args.steps, args.warmup, args.seed)
    cpu = None if args.no_cpu else cpu_baseline(head["workload"], fixed)
    del head["workload"]
    torch.cuda.empty_cache()

    value = head["kv_bytes"] / head["seconds"] / 1e9
    achieved = head["call_bytes"] / head["seconds"] / 1e9
    traffic = traffic_per_launch()
    line = {
        "metric": "KV-read GB/s (% HBM peak) + µs per decode-attn call, Llama-3-8B B=32 L=4096",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["seconds"] * 1e3, 5),
        "us_per_call": round(head["seconds"] * 1e6, 2),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic",
        "config": {
            "workload": "fp8 e4m3 paged decode attention (per-head scales), Llama-3-8B decode shape",
            "batch": BATCH, "q_len": 1, "q_heads": Q_HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM,
            "seq_len": 4096, "page_size": PAGE, "kv_bytes_per_call": head["kv_bytes"],
            "input_copies": head["copies"],
            "compute": "bf16 x bf16 MFMA for q.k, fp16 x fp16 MFMA for p.v, fp32 accumulation",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_attention_kernel",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": head["call_bytes"],
            "us_per_launch": round(head["seconds"] * 1e6, 2),
        },
        "ragged": None if ragged is None else {
            "lens": "uniform [1024, 8192], seed 100",
            "sum_len": int(sum(ragged_lens)),
            "us_per_call": round(ragged["seconds"] * 1e6, 2),
            "kv_gb_s": round(ragged["kv_bytes"] / ragged["seconds"] / 1e9, 1),
            "hbm_frac": round(ragged["kv_bytes"] / ragged["seconds"] / 1e9 / HBM_PEAK_GBS, 4),
        },
        "cpu_baseline": cpu,
        "paths": paths,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
