"""ctypes binding of ``libeconomize_amd.so`` (the C ABI of include/economize_amd.h).

The library is loaded on first use and never replaced by anything else: if it is missing, every entry point raises
``RuntimeError`` (build it with ``python -m economize_amd._build``). Nonzero return codes become :class:`ConfigError`
(validation, code 1) or ``RuntimeError`` (a failed launch, code 2) carrying ``eco_last_error()``.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

from .errors import ConfigError

LIBRARY = Path(__file__).resolve().with_name("libeconomize_amd.so")

ECO_BF16, ECO_FP8_E4M3, ECO_FP8_E5M2, ECO_FP16, ECO_FP32 = 0, 1, 2, 3, 4

_FORMATS = {
    torch.bfloat16: ECO_BF16,
    torch.float8_e4m3fn: ECO_FP8_E4M3,
    torch.float8_e5m2: ECO_FP8_E5M2,
    torch.float16: ECO_FP16,
    torch.float32: ECO_FP32,
}

# argument types of every exported function (kept in the order of include/economize_amd.h)
_P, _I, _L, _F, _S = c_void_p, c_int32, c_int64, c_float, c_size_t
_MASK = [_P, _L, _L, _L, _I]  # packed mask bits, word strides (batch, head, query), words per row
_PAGED_ARGS = [_P, _L, _L, _L, _P, _P, _I, _I, _P, _P, _P, _L, _I, _P, _P, _L, _L, _I, _I, _P, _P, _P, _L, _L, _L,
               _I, _I, _I, _I, _I, _I, _I, _F, _F] + _MASK
_PAGED_DECODE = _PAGED_ARGS[:1] + [_I] + _PAGED_ARGS[1:] + [_P, _S, _P]  # (the query's format after the query)
SIGNATURES: dict[str, tuple[type | None, list]] = {
    "eco_last_error": (ctypes.c_char_p, []),
    "eco_abi_version": (c_int32, []),
    "eco_paged_append": (c_int32, [_P, _P, _I, _L, _L, _L, _L, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "eco_paged_append_quest": (c_int32, [_P, _P, _I, _L, _L, _L, _L, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P,
                                         _P, _L, _I, _P, _P, _P, _P, _I, _P, _P, _L, _L, _L, _I, _I, _P]),
    "eco_fp8_encode": (c_int32, [_P, _I, _L, _L, _L, _P, _I, _L, _L, _L, _I, _I, _I, _I, _P, _P, _L, _L, _L, _P]),
    "eco_kv_head_absmax": (c_int32, [_P, _I, _I, _I, _I, _I, _L, _L, _L, _L, _P, _P]),
    "eco_fp8_scales_from_absmax": (c_int32, [_P, _I, _I, _P, _P]),
    "eco_paged_decode_workspace_size": (c_size_t, [_I, _I, _I, _I, _I, _I, _I, _I, _I]),
    "eco_paged_decode": (c_int32, _PAGED_DECODE),
    "eco_paged_decode_static": (c_int32, _PAGED_ARGS + [_P]),
    "eco_mask_bits": (c_int32, [_P, _L, _L, _L, _L, _I, _I, _I, _I, _P, _I, _P]),
    "eco_paged_gather": (c_int32, [_P, _P, _I, _I, _P, _P, _P, _L, _I, _P, _P, _I, _L, _L, _L, _L, _L, _L, _I, _I, _I,
                                   _I, _I, _P]),
    "eco_kivi_gather": (c_int32, [_P, _I, _P, _P, _I, _P, _P, _P, _L, _I, _P, _P, _I, _L, _L, _L, _L, _L, _L, _I, _I, _I,
                                  _I, _I, _I, _P]),
    "eco_decode_workspace_size": (c_size_t, [_I, _I, _I, _I, _I, _I, _I]),
    "eco_gathered_decode": (c_int32, [_P, _I, _L, _L, _L, _P, _P, _L, _L, _L, _L, _L, _L,  # q .. value strides
                                      _P, _P, _L, _L, _L, _L, _L, _L, _P, _L, _L, _P, _P, _I, _I,  # compact entries
                                      _P, _L, _L, _L, _L, _P, _P, _L, _L, _L,  # mask, sinks, out
                                      _I, _I, _I, _I, _I, _I, _I, _F, _F, _P, _S, _P]),
    "eco_decode": (c_int32, [_P, _I, _L, _L, _L, _P, _P, _I, _L, _L, _L, _L, _L, _L, _P, _P, _P, _L, _L, _L, _L, _P, _P,
                             _L, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _F, _P, _S, _P]),
    "eco_quest_page_bounds": (c_int32, [_P, _I, _I, _P, _L, _I, _I, _I, _I, _P, _P, _L, _L, _L, _I, _I, _I, _I, _P]),
    "eco_quest_select_workspace_size": (c_size_t, [_I, _I, _I]),
    "eco_kivi_block_bytes": (c_size_t, [_I, _I, _I]),
    "eco_kivi_schedule": (c_int32, [_P, _I, _I, _P, _P, _P, _I, _P]),
    "eco_kivi_fake_quantize": (c_int32, [_P, _I, _L, _L, _L, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "eco_kivi_pack_quantize": (c_int32, [_I, _P, _I, _L, _L, _L, _I, _I, _P, _L, _L, _L, _P, _P, _L, _L, _L, _P, _P,
                                         _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "eco_kivi_packed_gather": (c_int32, [_I, _P, _L, _L, _L, _P, _P, _L, _L, _L, _P, _P, _L, _L, _L, _I, _P, _I, _L, _L,
                                         _L, _I, _I, _I, _I, _I, _I, _P]),
    "eco_kivi_cells_layout": (c_int32, [_I, _I, _I, _I, _P]),
    "eco_kivi_cells_quantize": (c_int32, [_P, _I, _L, _L, _L, _I, _I, _I, _P, _L, _I, _P, _P, _P, _I, _I, _I, _I, _I,
                                          _P, _P]),
    "eco_kivi_cells_attention_workspace_size": (c_size_t, [_I, _I, _I, _I, _I, _I]),
    "eco_kivi_cells_attention": (c_int32, [_P, _L, _L, _P, _I, _L, _L, _L, _I, _I, _I, _P, _L, _I, _P, _P, _I, _I, _I,
                                           _I, _I, _I, _P, _P, _L, _L, _I, _F, _F, _P, _S, _P]),
    "eco_kivi_cells_clear_flags": (c_int32, [_P, _I, _L, _L, _L, _I, _I, _I, _P, _I, _I, _I, _I, _P]),
    "eco_kivi_quantize": (c_int32, [_I, _P, _I, _L, _L, _L, _L, _I, _I, _P, _P, _P, _I, _P, _L, _I, _I, _I, _I, _I, _I,
                                    _I, _P, _P]),
    "eco_kivi_ring_write": (c_int32, [_P, _P, _I, _L, _L, _L, _L, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P]),
    "eco_kivi_decode_workspace_size": (c_size_t, [_I, _I, _I, _I, _I, _I, _I]),
    "eco_kivi_decode": (c_int32, [_P, _L, _L, _L, _P, _I, _P, _P, _I, _P, _P, _P, _L, _I, _P, _P, _P, _L, _L, _L, _I, _I,
                                  _I, _I, _I, _I, _I, _I, _F, _F] + _MASK + [_P, _S, _P]),
    "eco_quest_refresh_bounds": (c_int32, [_P, _I, _I, _P, _L, _I, _P, _P, _P, _I, _P, _P, _L, _L, _L, _I, _I, _I, _I,
                                           _I, _P]),
    "eco_quest_select": (c_int32, [_P, _I, _L, _L, _L, _P, _P, _I, _L, _L, _L, _P, _I, _I, _I, _P, _I, _I, _I, _I, _I,
                                   _P, _S, _P]),
    "eco_quest_dense_bounds": (c_int32, [_P, _I, _L, _L, _L, _I, _I, _I, _I, _P, _P, _I, _L, _L, _L, _I, _I, _I, _P]),
    "eco_quest_decode_workspace_size": (c_size_t, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I]),
    "eco_quest_decode": (c_int32, [_P, _I, _L, _L, _L, _P, _P, _I, _L, _L, _L, _L, _L, _L, _P, _P,  # q .. scales
                                   _P, _L, _L, _I, _P, _I, _I,  # index, pages, done, page size, min_done
                                   _P, _L, _L, _L, _L, _P, _P, _L, _L, _L,  # mask, sinks, out
                                   _I, _I, _I, _I, _I, _I, _I, _F, _F, _P, _S, _P]),
    "eco_kivi_packed_decode": (c_int32, [_P, _I, _L, _L, _L, _P, _P, _L, _L, _L, _L, _L, _L, _I,  # q .. ring
                                         _P, _L, _L, _L, _P, _P, _L, _L, _L,  # key codes, scales, zero points
                                         _P, _L, _L, _L, _P, _P, _L, _L, _L,  # value codes, scales, zero points
                                         _P, _P, _I, _I, _I,  # counts, bits, groups
                                         _P, _L, _L, _L, _L, _P, _P, _L, _L, _L,  # mask, sinks, out
                                         _I, _I, _I, _I, _I, _I, _I, _F, _F, _P, _S, _P]),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (``RuntimeError`` if it is not built)."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY.name} is not built: run `python -m economize_amd._build`")
        handle = ctypes.CDLL(str(LIBRARY))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call ``name`` and raise on a nonzero return code."""
    rc = getattr(lib(), name)(*args)
    if rc:
        message = (lib().eco_last_error() or b"").decode()
        if rc == 1:
            raise ConfigError(message)
        raise RuntimeError(message)


def fmt(dtype: torch.dtype) -> int:
    """The C-ABI element format of a torch dtype."""
    try:
        return _FORMATS[dtype]
    except KeyError:
        raise ConfigError(f"no kernel element format for {dtype}") from None


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def stream_of(device: torch.device) -> int:
    """The current HIP stream of ``device`` (the reference launches on it too, attention/decode.py:318)."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """The device all ``tensors`` live on; they must be on one GPU (there is no CPU path)."""
    device = tensors[0].device
    if device.type != "cuda":
        raise RuntimeError("economize_amd kernels run on an AMD GPU; the tensors are on " + str(device))
    for t in tensors[1:]:
        if t is not None and t.device != device:
            raise ConfigError(f"tensors on {t.device} and {device}")
    return device
