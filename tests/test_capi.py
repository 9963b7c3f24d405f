"""The C ABI on the CPU: the library builds and exports every function include/economize_amd.h declares, and the
kernels' fp8 / bf16 encoders (compiled for the host) agree bit for bit with the oracle."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import fp8 as ofp8
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits

ROOT = Path(__file__).resolve().parents[1]


def _declared() -> list[str]:
    names = []
    for header in (ROOT / "include").glob("*.h"):
        names += re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(eco_\w+)\s*\(", header.read_text(), flags=re.M)
    return sorted(set(names))


def _library() -> Path:
    from economize_amd import _build

    if not _build.LIBRARY.exists():
        _build.build()
    return _build.LIBRARY


def test_library_exports_every_declared_function() -> None:
    declared = _declared()
    assert "eco_paged_decode" in declared and "eco_last_error" in declared
    handle = ctypes.CDLL(str(_library()))
    missing = [name for name in declared if not hasattr(handle, name)]
    assert not missing
    from economize_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared  # the binding declares every entry point
    assert _lib.lib().eco_abi_version() == 8


def _parameter_counts() -> dict[str, int]:
    counts = {}
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        for name, params in re.findall(r"\b(eco_\w+)\s*\(([^)]*)\)\s*;", text):
            params = params.strip()
            counts[name] = 0 if params in ("", "void") else params.count(",") + 1
    return counts


def test_binding_argument_counts_match_the_header() -> None:
    from economize_amd import _lib

    counts = _parameter_counts()
    assert set(counts) == set(_lib.SIGNATURES)
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        assert len(argtypes) == counts[name], name


def test_validation_errors_are_reported_without_a_device() -> None:
    from economize_amd import _lib

    lib = _lib.lib()
    rc = lib.eco_paged_append(None, None, 0, 0, 0, 0, 0, None, 3, None, None, 1, 1, 64, 16, 1, None, None, None)
    assert rc == 1 and b"null" in lib.eco_last_error()
    assert lib.eco_paged_decode_workspace_size(32, 1, 32, 8, 128, 4096, 0, 16, 1) > 0


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_kernel_encoders_match_the_oracle(tmp_path: Path) -> None:
    exe = tmp_path / "codec"
    subprocess.run(["g++", "-O2", "-std=c++17", str(ROOT / "tests/native/fp8_codec_check.cpp"), "-o", str(exe)],
                   check=True)
    rng = np.random.default_rng(0)
    every_bf16 = bf16_bits_to_f32(np.arange(65536, dtype=np.uint16))
    rand = (rng.standard_normal(1 << 20) * np.exp2(rng.integers(-24, 16, 1 << 20))).astype(np.float32)
    x = np.concatenate([every_bf16[np.isfinite(every_bf16)], rand]).astype(np.float32)
    out = subprocess.run([str(exe)], input=x.tobytes(), capture_output=True, check=True).stdout
    got = np.frombuffer(out, dtype=np.uint8).reshape(-1, 4)
    for col, fmt in ((0, "e4m3"), (1, "e5m2")):
        limit = np.float32(ofp8.FORMATS[fmt][3])
        inside = np.abs(x) <= limit  # the kernels clamp before encoding, as fp8.py:84-86
        assert np.array_equal(got[inside, col], ofp8.fp8_encode(x[inside], fmt, None))
    assert np.array_equal(got[:, 2:].copy().view(np.uint16).ravel(), f32_to_bf16_bits(x))
