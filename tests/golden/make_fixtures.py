"""Write ``reference_golden.npz`` beside this script from the reference's own golden data files.

The reference commits the outputs of its golden cases as tensor files (tests/golden/data/*.pt, written by its
tests/golden/regenerate.py from the cases of tests/golden/catalog.py). This script copies the ones this path covers
into one numpy archive, reading them with ``torch.load(..., weights_only=True)`` (nothing in the files is executed):

* ``dense_logits`` ``[2, 24, 128]`` float32: the base model's logits on the held-out sequence (catalog.py:41-45), which
  pins the model recipe every other case builds on;
* ``kv_fp8_tokens``, ``kv_kivi_2bit_tokens``, ``kv_quest_tokens`` ``[24]`` int64: greedy tokens after the 16-token
  prompt under ``FP8KVConfig()``, ``KIVIConfig(bits=2, group_size=4, residual_length=8)`` and
  ``QuestConfig(page_size=16, token_budget=32, dense_layers=0)`` (catalog.py:163-170, 195-207).

Run from the repository root: ``python tests/golden/make_fixtures.py [reference root]``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

CASES = {"dense": "logits", "kv_fp8": "tokens", "kv_kivi_2bit": "tokens", "kv_quest": "tokens"}


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    arrays = {}
    for name, key in CASES.items():
        tensors = torch.load(root / "tests" / "golden" / "data" / f"{name}.pt", weights_only=True)
        arrays[f"{name}_{key}"] = tensors[key].numpy()
    out = Path(__file__).resolve().parent / "reference_golden.npz"
    np.savez_compressed(out, **arrays)
    print(f"wrote {out}: " + ", ".join(f"{k} {v.dtype} {v.shape}" for k, v in arrays.items()))


if __name__ == "__main__":
    main()
