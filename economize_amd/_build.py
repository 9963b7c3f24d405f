"""Builds ``libeconomize_amd.so`` (the HIP kernels and their C ABI) for gfx950 with ``hipcc``, in-tree.

Run ``python -m economize_amd._build`` or call :func:`build`. Every HIP source is compiled with

* ``--offload-arch=gfx950`` (MI355X only),
* ``-ffp-contract=off`` (no fused multiply-add unless a kernel asks for one: the reference rounds products and sums
  separately wherever it fixes an order, attention/_libdevice.py:1-60),
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` (no packed fp32 VALU instructions).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIBRARY = HERE / "libeconomize_amd.so"
SOURCES = ["capi.hip", "paged_attention.hip", "paged_attention_f16.hip", "kv_quant.hip", "quest.hip", "kivi.hip", "dense_attention.hip", "gather.hip",
           "kivi_dense.hip", "kivi_cells.hip", "kivi_verify.hip", "kivi_packed.hip"]

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _compile(source: str, build_dir: Path) -> Path:
    obj = build_dir / (Path(source).stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(CSRC / source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    errors = [line for line in result.stderr.splitlines() if "packed-fp32-ops" not in line]
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n" + "\n".join(errors))
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library next to this file; returns its path."""
    build_dir = HERE / "_build"
    build_dir.mkdir(exist_ok=True)
    workers = min(len(SOURCES), max(1, (os.cpu_count() or 1)))
    with ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(lambda s: _compile(s, build_dir), SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError("linking libeconomize_amd.so failed:\n" + result.stderr)
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
