"""Write ``quest_select_vectors.npz`` beside this script: Quest page selections computed by the reference's own
``page_bounds`` and ``select_pages`` (src/economize/attention/quest.py:54-65, 73-108) on the CPU.

The reference's selection is plain torch (two einsums, ``masked_fill``, ``topk``, a sort), so its CPU result on
seeded inputs is a set of vectors for this path: the bounds and query go in, the selected page indices come out.
Nothing of the reference ships with the vectors; the archive holds only inputs and outputs:

* ``{case}_query`` uint16 bf16 bits ``[B, Hq, Q, D]``, ``{case}_kmin`` / ``{case}_kmax`` uint16 bf16 bits
  ``[B, Hkv, P, D]`` (the reference's ``page_bounds`` of seeded keys, or constructed bounds),
  ``{case}_done`` int32 ``[B]``, ``{case}_meta`` int64 ``[max_done, pages]``;
* ``{case}_index`` int32 ``[B, Hkv, pages]``: the reference's selection.

Exact ties (equal fp32 scores) are where the reference's ``torch.topk`` keeps pages in an unspecified order: on the
CPU it keeps higher-index pages of a tied group as well as lower ones, while this path breaks ties toward the lower
page index. The tests compare those cases by the scores selected, not by the indices.

Cases: random keys at head dims 64 and 128, fp8 e4m3 keys (bounds in bf16), several query rows per KV head, a
scaled-down planted workload (32 pages per row whose keys are the query plus 0.1 N(0, 1)), rows whose committed pages
number at most the budget, pages of identical bounds (exact ties), and near ties: pages that differ from a common
base in one small channel by a few bf16 units, so that their exact scores differ by about one fp32 unit of the score.

Run from the repository root, in a container that holds the reference (it imports the reference):
``python tests/golden/make_quest_vectors.py [reference root]``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

PAGE = 16


def bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def keyed_case(page_bounds, gen, batch, q_heads, kv_heads, queries, dim, pages_total, dtype=torch.bfloat16,
               planted=0):
    query = torch.randn(batch, q_heads, queries, dim, generator=gen).to(torch.bfloat16)
    keys = torch.randn(batch, kv_heads, pages_total * PAGE, dim, generator=gen)
    if planted:
        ref = query.float().unflatten(1, (kv_heads, -1))[:, :, 0, 0]  # [B, Hkv, D]: the group's first query row
        for b in range(batch):
            for h in range(kv_heads):
                chosen = torch.randperm(pages_total, generator=gen)[:planted]
                for p in chosen.tolist():
                    keys[b, h, p * PAGE:(p + 1) * PAGE] = ref[b, h] + 0.1 * torch.randn(PAGE, dim, generator=gen)
    keys = keys.to(dtype)
    kmin, kmax = page_bounds(keys, 0, pages_total, PAGE)
    return query, kmin, kmax


def constructed_case(gen, batch, q_heads, kv_heads, dim, pages_total, mode):
    """Bounds built directly: ``ties`` repeats every page three times; ``near`` gives every page a common base and
    moves one small channel's minimum and maximum by up to three bf16 units."""
    query = torch.randn(batch, q_heads, 1, dim, generator=gen).to(torch.bfloat16)
    if mode == "ties":
        distinct = -(-pages_total // 3)
        lo = torch.randn(batch, kv_heads, distinct, dim, generator=gen)
        hi = lo + torch.rand(batch, kv_heads, distinct, dim, generator=gen) * 2
        kmin = lo.repeat_interleave(3, dim=2)[:, :, :pages_total].to(torch.bfloat16)
        kmax = hi.repeat_interleave(3, dim=2)[:, :, :pages_total].to(torch.bfloat16)
        return query, kmin, kmax
    lo = torch.randn(batch, kv_heads, 1, dim, generator=gen)
    hi = lo + torch.rand(batch, kv_heads, 1, dim, generator=gen) * 2
    # one channel of every (row, KV head) holds a small bound (about 2e-3), so that a bf16 unit there moves the
    # page's score by about one fp32 unit of the whole score: the pages' scores then differ in their last bits only,
    # where the summation order decides the rounding
    channel = torch.randint(0, dim, (batch, kv_heads), generator=gen)
    for b in range(batch):
        for h in range(kv_heads):
            small = 2e-3 * (1 + torch.rand(1, generator=gen))
            lo[b, h, 0, channel[b, h]] = small
            hi[b, h, 0, channel[b, h]] = small * 1.5
    base_lo = lo.to(torch.bfloat16).expand(-1, -1, pages_total, -1).contiguous()
    base_hi = hi.to(torch.bfloat16).expand(-1, -1, pages_total, -1).contiguous()
    lo_bits = base_lo.view(torch.int16).clone()
    hi_bits = base_hi.view(torch.int16).clone()
    for b in range(batch):
        for h in range(kv_heads):
            c = int(channel[b, h])
            for p in range(pages_total):
                lo_bits[b, h, p, c] += int(torch.randint(-3, 4, (1,), generator=gen))
                hi_bits[b, h, p, c] += int(torch.randint(-3, 4, (1,), generator=gen))
    return query, lo_bits.view(torch.bfloat16), hi_bits.view(torch.bfloat16)


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(root / "src"))
    from economize.attention.quest import page_bounds, select_pages

    gen = torch.Generator().manual_seed(2024)
    cases = {
        # name: (query, kmin, kmax, done, pages)
    }
    q, lo, hi = keyed_case(page_bounds, gen, 3, 8, 2, 1, 128, 64)
    cases["random_d128"] = (q, lo, hi, [64, 40, 5], 16)
    q, lo, hi = keyed_case(page_bounds, gen, 2, 8, 4, 1, 64, 48)
    cases["random_d64"] = (q, lo, hi, [48, 33], 8)
    q, lo, hi = keyed_case(page_bounds, gen, 2, 8, 2, 1, 128, 40, dtype=torch.float8_e4m3fn)
    cases["fp8_keys"] = (q, lo, hi, [40, 39], 12)
    q, lo, hi = keyed_case(page_bounds, gen, 2, 16, 2, 4, 128, 50)
    cases["four_queries"] = (q, lo, hi, [50, 21], 10)
    q, lo, hi = keyed_case(page_bounds, gen, 2, 8, 2, 1, 128, 128, planted=32)
    cases["planted"] = (q, lo, hi, [128, 127], 48)
    q, lo, hi = keyed_case(page_bounds, gen, 3, 4, 2, 1, 128, 20)
    cases["short_rows"] = (q, lo, hi, [20, 6, 0], 8)
    q, lo, hi = constructed_case(gen, 2, 8, 2, 128, 60, "ties")
    cases["exact_ties"] = (q, lo, hi, [60, 45], 11)
    q, lo, hi = constructed_case(gen, 2, 8, 2, 128, 80, "near")
    cases["near_ties"] = (q, lo, hi, [80, 80], 20)

    arrays = {}
    for name, (query, kmin, kmax, done, pages) in cases.items():
        done_t = torch.tensor(done, dtype=torch.int32)
        max_done = max(done)
        index = select_pages(query, kmin, kmax, done_t, max_done, pages)
        arrays[f"{name}_query"] = bits(query)
        arrays[f"{name}_kmin"] = bits(kmin)
        arrays[f"{name}_kmax"] = bits(kmax)
        arrays[f"{name}_done"] = done_t.numpy()
        arrays[f"{name}_meta"] = np.array([max_done, pages], dtype=np.int64)
        arrays[f"{name}_index"] = index.numpy().astype(np.int32)
    out = Path(__file__).resolve().parent / "quest_select_vectors.npz"
    np.savez_compressed(out, **arrays)
    print(f"wrote {out}: {len(cases)} cases, {out.stat().st_size} bytes")


if __name__ == "__main__":
    main()
