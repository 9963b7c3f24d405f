"""CPU oracle of economize's compressed-KV decode-attention path (test infrastructure only).

This package restates, in numpy, the algorithms of the reference (Thiggel/economize 0.6.0) that the HIP kernels of
``economize_amd`` implement: fp8 encode/decode with scales, KIVI quantization, packing and schedule, the fp32
attention definition, Quest page bounds and page selection, and the paged-cache gathers used to compare a paged
kernel with the contiguous definition. Every function cites the reference file and lines it follows.

It is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import it. The product path (``economize_amd``) never imports, calls or falls back to anything here.

Pinning (how each function is checked independently of its own formula) is listed per module in its docstring.
Functions whose exact bits no independent check fixes say "parity unpinned" there.
"""

from . import attention, fp8, kivi, numerics, paged, quest  # noqa: F401
