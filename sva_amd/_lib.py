"""ctypes binding of the gfx950 C-ABI library (include/sva_hip.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already mapped (one libamdhip64 per process).  There is no CPU
fallback: if the library is missing, or a tensor is not on a ROCm device, the
call raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsva_hip.so"

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# argument signatures of include/sva_hip.h
_SIGNATURES: dict[str, tuple[type, list]] = {
    "sva_abi_version": (_I, []),
    "sva_last_error": (ctypes.c_char_p, []),
    "sva_write_encode": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64,
                              _P, _I, _I64, _P]),
    "sva_write_encode_batch": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                    _P, _P, _P, _I64, _I64, _P, _I, _I64, _P]),
    "sva_query_lut": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I,
                           _I64, _I64, _I64, _P, _P, _P, _P]),
    "sva_pq_scores": (_I, [_P, _P, _I, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "sva_summon_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "sva_summon": (_I, [_P, _P, _P, _P, _I, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                        _P, _I, _I64, _P, _P, _P, _P, _SZ, _P]),
    "sva_summon_select": (_I, [_P, _P, _P, _P, _I, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                               _I64, _P, _I, _I64, _P, _P, _P, _I64, _P, _P, _P, _SZ, _P]),
    "sva_lookup_select": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I, _I64, _P, _I64, _I64,
                               _I64, _P, _I, _I64, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _SZ, _P]),
    "sva_lookup_verify": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I, _I64, _P, _I64, _I64,
                               _I64, _P, _I, _I64, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _SZ,
                               _P, _P, _I, _I64, _I64, _I64, _F, _P, _I, _I64, _P, _SZ, _P, _P]),
    "sva_summon_strategy": (_I, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I]),
    "sva_budget_select": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P]),
    "sva_verify_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "sva_postings_build": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "sva_inverted_slots": (_I64, [_I64, _I64, _I64, _I64]),
    "sva_inverted_candidates": (_I, [_P, _P, _P, _I64, _P, _I, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                     _I64, _P, _I, _I, _P, _P, _I64, _P]),
    "sva_unique_select_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "sva_unique_refill_select": (_I, [_P, _P, _I64, _I64, _I, _I64, _I64, _I64, ctypes.c_double, ctypes.c_double,
                                      _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _SZ, _P]),
    "sva_postings_build_ragged": (_I, [_P, _I, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "sva_inverted_slots_ragged": (_I64, [_I64, _I64, _I64]),
    "sva_inverted_candidates_ragged": (_I, [_P, _P, _P, _I64, _P, _I, _I64, _P, _P, _I64, _P, _P, _P, _I64, _I64,
                                            _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "sva_unique_refill_select_ragged": (_I, [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_double,
                                             ctypes.c_double, _I64, _P, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P,
                                             _P, _SZ, _P]),
    "sva_centroid_update": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "sva_key_weights": (_I, [_P, _P, _I64, _I64, _I64, _F, _P, _P]),
    "sva_residual_adapter": (_I, [_P, _I, _I64, _P, _I, _I64, _P, _P, _F, _I64, _I64, _I64, _P, _I, _I64, _P]),
    "sva_top_unique_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "sva_top_unique": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _SZ, _P]),
    "sva_verify": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _I, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _I64,
                        _I64, _I64, _I64, _F, _P, _I, _I64, _I64, _I64, _P, _SZ, _P]),
    "sva_stream_read_sink_words": (_I64, [_I64]),
    "sva_stream_read": (_I, [_P, _I64, _P, _I64, _P]),
    "sva_verify_noalloc": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _I, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _I64,
                                _I64, _I64, _I64, _I64, _F, _P, _I, _I64, _I64, _I64, _P]),
    "sva_decode_layer_create": (_I, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _F,
                                     ctypes.POINTER(_P)]),
    "sva_decode_layer_bind": (_I, [_P, _P, _I64, _P, _I, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P, _SZ,
                                   _P]),
    "sva_decode_layer_step": (_I, [_P, _P, _I, _I64, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _I, _I64, _P]),
    "sva_decode_layer_destroy": (None, [_P]),
}


class SVAKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """Load libsva_hip.so once; raise if it has not been built."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise SVAKernelError(
                    f"{LIB_PATH} is missing: build it with `python -m sva_amd.build` (hipcc, gfx950). "
                    "The SVA decode path has no CPU fallback."
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(status: int, name: str) -> None:
    if status != 0:
        msg = lib().sva_last_error().decode("utf-8", "replace")
        raise SVAKernelError(f"{name} failed (status {status}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The current HIP stream of `device` as an integer handle (the raw
    accessor skips building a torch Stream object: a few microseconds per
    call on the decode path)."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
CODE_TYPES = {torch.uint8: 0, torch.int16: 1, torch.int32: 2, torch.int64: 3}
MASK_TYPES = {None: 0, torch.float32: 1, torch.bfloat16: 2, torch.float16: 3, torch.bool: 4}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError as exc:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from exc


def code_type(t: torch.Tensor) -> int:
    try:
        return CODE_TYPES[t.dtype]
    except KeyError as exc:
        raise TypeError(f"unsupported code dtype {t.dtype}; expected uint8, int16, int32 or int64") from exc


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""

    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "sva_amd runs its decode path only on a ROCm GPU (gfx950); got a tensor on "
                f"{t.device}. Move the model to the GPU; there is no CPU fallback."
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"tensors on different devices: {device} and {t.device}")
    if device is None:
        raise RuntimeError("no device tensor given")
    return device
