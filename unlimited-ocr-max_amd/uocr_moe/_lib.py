"""Loads ``libuocr_moe.so`` (the HIP library) and declares its C ABI (``include/uocr_moe.h``).

torch is imported first so that the library binds to the HIP runtime torch
already loaded, and device pointers and streams from torch are valid for it.
A missing library is an error: there is no CPU fallback on the product path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library links against)

LIB_PATH = Path(os.environ.get("UOCR_MOE_LIB", Path(__file__).resolve().parent / "libuocr_moe.so"))
ERRLEN = 512

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t
_cp = ctypes.c_char_p


class UocrError(RuntimeError):
    """A call the library refused; the message is the reference's text, ``"<op>: <reason>"``."""


class Layer(ctypes.Structure):
    """``uocr_moe_layer`` (include/uocr_moe.h)."""

    _fields_ = [
        ("num_experts", _i64), ("hidden", _i64), ("ffn", _i64), ("shared_ffn", _i64),
        ("top_k", _i64), ("group", _i64), ("int8", ctypes.c_int32), ("renormalize", ctypes.c_int32),
        ("router", _vp), ("gate_proj", _vp), ("up_proj", _vp), ("down_proj", _vp),
        ("gate_proj_scales", _vp), ("up_proj_scales", _vp), ("down_proj_scales", _vp),
        ("shared_gate", _vp), ("shared_up", _vp), ("shared_down", _vp),
    ]


# name -> argtypes (every entry point returns int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "uocr_moe_abi_version": [],
    "uocr_moe_int8_qmv": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
                          _vp, _cp, _sz],
    "uocr_moe_bf16_qmv": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _cp, _sz],
    "uocr_int8_dequant_expert": [_vp, _i64, _i64, _int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64,
                                 _vp, _cp, _sz],
    "uocr_quantize_per_group": [_vp, _vp, _vp, _int, _i64, _i64, _i64, _vp, _cp, _sz],
    "uocr_dense_bf16_qmv": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _cp, _sz],
    "uocr_ngram_block": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _cp, _sz],
    "uocr_paged_decode_attention_qkv": [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64,
                                        _i64, _i64, _vp, _i64, _vp, _i64, _vp, ctypes.c_float, _vp, _sz, _vp, _cp,
                                        _sz],
    "uocr_rms_norm_dense_bf16_qmv": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp, ctypes.c_float, _vp, _i64, _i64,
                                     _i64, _vp, _cp, _sz],
    "uocr_rms_norm": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp, _cp, _sz],
    "uocr_rope": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _cp, _sz],
    "uocr_swiglu": [_vp, _vp, _i64, _i64, _vp, _cp, _sz],
    "uocr_paged_attention_workspace_bytes": [_i64, _i64, _i64],
    "uocr_paged_decode_attention": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _i64,
                                    _vp, _i64, _vp, ctypes.c_float, _vp, _sz, _vp, _cp, _sz],
    "uocr_moe_workspace_bytes": [ctypes.POINTER(Layer), _i64, _int],
    "uocr_moe_gate": [_vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _int, _vp, _sz, _vp, _cp, _sz],
    "uocr_moe_decode_rows": [_vp, _vp, _i64, _i64, ctypes.POINTER(Layer), _vp, _vp, _vp, _sz, _vp, _cp, _sz],
    "uocr_moe_decode_rows_static": [_vp, _vp, _i64, _i64, ctypes.POINTER(Layer), _vp, _vp, _vp, _cp, _sz],
    "uocr_moe_decode_stack": [_vp, _vp, _i64, _i64, ctypes.POINTER(ctypes.POINTER(Layer)), _i64, _vp, _cp, _sz],
    "uocr_moe_forward": [_vp, _vp, _i64, _i64, ctypes.POINTER(Layer), _vp, _vp, _vp, _sz, _vp, _cp, _sz],
    "uocr_moe_release": [],
    "uocr_moe_timing_begin": [_int, _cp, _sz],
    "uocr_moe_fused_errors": [_vp, ctypes.POINTER(ctypes.c_uint32), _cp, _sz],
    "uocr_moe_fused_status": [_vp, _vp, _cp, _sz],
    "uocr_moe_fused_trace": [_vp, _i64, ctypes.POINTER(_int), _cp, _sz],
    "uocr_moe_timing_end": [_int, _vp, _vp, _sz, ctypes.POINTER(_int), _cp, _sz],
}
_RESTYPES = {"uocr_moe_workspace_bytes": _sz, "uocr_paged_attention_workspace_bytes": _sz, "uocr_moe_release": None}

_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The library with its signatures declared; raises if it was not built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP library first (python __graft_entry__.py or "
                "unlimited-ocr-max_amd/build.py); there is no CPU fallback"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, _int)
        _LIB = lib
    return _LIB


def call(name: str, *args) -> None:
    """Calls an entry point that takes a trailing ``(err, errlen)`` and raises its message on failure."""
    err = ctypes.create_string_buffer(ERRLEN)
    rc = getattr(load(), name)(*args, err, ERRLEN)
    if rc != 0:
        raise UocrError(err.value.decode() or f"{name} failed with code {rc}")


def timing_begin(capacity: int) -> None:
    """Records a start/stop event pair around each of the next ``capacity`` kernel launches."""
    call("uocr_moe_timing_begin", int(capacity))


def timing_end(capacity: int) -> list[tuple[str, float]]:
    """``[(kernel name, ms)]`` of the launches recorded since :func:`timing_begin`, in order."""
    import numpy as np

    ms = np.zeros(capacity, np.float32)
    names = ctypes.create_string_buffer(capacity * 32)
    count = _int(0)
    call("uocr_moe_timing_end", int(capacity), ms.ctypes.data, ctypes.addressof(names), 32, ctypes.byref(count))
    raw = names.raw
    return [(raw[i * 32 : (i + 1) * 32].split(b"\0", 1)[0].decode(), float(ms[i])) for i in range(count.value)]


def fused_errors(stream: int | None = None) -> int:
    """Synchronises ``stream`` (default: torch's current) and returns the persistent decode kernel's error word
    (1: a launch ran out of its bounded waits; its slot, poisoned until now, is cleared by this call)."""
    import torch

    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    v = ctypes.c_uint32(0)
    call("uocr_moe_fused_errors", stream, ctypes.byref(v))
    return int(v.value)
