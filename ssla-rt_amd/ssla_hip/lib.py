"""ctypes binding of libssla_hip.so (include/ssla_hip.h).

The library is built in-tree (ssla-rt_amd/Makefile, or __graft_entry__.build)
and loaded from ssla-rt_amd/libssla_hip.so.  There is no fallback: if the
library is missing, load() raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

from . import abi

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_ROOT / "libssla_hip.so"

SSLA_OK = 0

# name -> (restype, argtypes); exactly the entry points of include/ssla_hip.h
_VP, _I, _LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
_FP, _UP = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint)
_SIGNATURES = {
    "ssla_hip_last_error": (ctypes.c_char_p, []),
    "ssla_hip_abi_layout": (_I, [ctypes.POINTER(_LL), _I]),
    "ssla_hip_malloc_device": (_I, [ctypes.c_size_t, ctypes.POINTER(_VP)]),
    "ssla_hip_malloc_host": (_I, [ctypes.c_size_t, ctypes.POINTER(_VP)]),
    "ssla_hip_free_device": (_I, [_VP]),
    "ssla_hip_free_host": (_I, [_VP]),
    "ssla_hip_memcpy": (_I, [_VP, _VP, ctypes.c_size_t]),
    "ssla_hip_memset": (_I, [_VP, _I, ctypes.c_size_t]),
    "ssla_hip_device_synchronize": (_I, []),
    "ssla_hip_stream_create": (_I, [ctypes.POINTER(_VP)]),
    "ssla_hip_stream_destroy": (_I, [_VP]),
    "ssla_hip_stream_synchronize": (_I, [_VP]),
    "ssla_hip_npz_read": (_LL, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                                _LL, ctypes.POINTER(_LL), ctypes.POINTER(_I)]),
    "ssla_hip_meta_read": (_I, [ctypes.c_char_p, ctypes.POINTER(_I)]),
    "ssla_hip_model_load": (_I, [ctypes.c_char_p, ctypes.POINTER(_VP)]),
    "ssla_hip_model_info": (_I, [_VP, ctypes.POINTER(abi.SslaHipModelInfo)]),
    "ssla_hip_model_free": (None, [_VP]),
    "ssla_hip_config_bind": (_I, [_VP, _I, ctypes.POINTER(abi.HybridS2S3Config)]),
    "ssla_hip_state_alloc": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _I]),
    "ssla_hip_state_reset": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _I]),
    "ssla_hip_state_reset_async": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _I, _VP]),
    "ssla_hip_state_free": (None, [ctypes.POINTER(abi.HybridS2S3Config), _I]),
    "ssla_hip_preds_alloc": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _I]),
    "ssla_hip_preds_free": (None, [ctypes.POINTER(abi.HybridS2S3Config), _I]),
    "ssla_hip_drain_n": (_I, [ctypes.POINTER(abi.HybridS2S3Config), ctypes.POINTER(_VP),
                              ctypes.POINTER(_I), ctypes.POINTER(_VP), ctypes.POINTER(_VP)]),
    "ssla_hip_drain_n2": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _VP, _VP, _I, _I, _VP, _VP]),
    "ssla_hip_drain_n_ex": (_I, [ctypes.POINTER(abi.HybridS2S3Config), ctypes.POINTER(_VP),
                                 ctypes.POINTER(_I), ctypes.POINTER(_VP),
                                 ctypes.POINTER(abi.SslaHipDrainOpts)]),
    "ssla_hip_drain_reserve": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _I]),
    "ssla_hip_drain_batch_noalloc": (_I, [ctypes.POINTER(abi.HybridS2S3Config),
                                          ctypes.POINTER(_VP), ctypes.POINTER(_I),
                                          ctypes.POINTER(_VP), ctypes.POINTER(_VP), _I, _VP, _I]),
    "ssla_hip_wall_clock_khz": (_I, [ctypes.POINTER(_I)]),
    "ssla_hip_timing_alloc": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _I, ctypes.c_uint]),
    "ssla_hip_timing_free": (None, [ctypes.POINTER(abi.HybridS2S3Config), _I]),
    "ssla_hip_persistent_start": (_I, [ctypes.POINTER(abi.HybridS2S3Config), ctypes.POINTER(_VP),
                                       ctypes.c_ulonglong, ctypes.POINTER(_VP), _VP,
                                       ctypes.POINTER(_VP), ctypes.c_uint,
                                       ctypes.POINTER(abi.SslaHipLiveOpts), ctypes.POINTER(_VP)]),
    "ssla_hip_persistent_start2": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _VP, _VP,
                                        ctypes.c_ulonglong, _VP, _VP, _VP, _VP, _VP,
                                        ctypes.c_uint, ctypes.POINTER(_VP)]),
    "ssla_hip_persistent_wait": (_I, [_VP, _I, ctypes.POINTER(_I)]),
    "ssla_hip_preds_snapshot": (_I, [_FP, _UP, _I, _I, _FP, _UP, _I]),
    "ssla_hip_decode_cells": (_I, [_FP, _I, _I, _I, _I, _I, _I, _I, _FP]),
    "ssla_hip_grid_decode": (_I, [ctypes.POINTER(abi.HybridS2S3Config), _FP, _I, _I, _I, _FP]),
    "ssla_hip_collect_boxes": (_I, [_FP, _I, _I, _I, _I, ctypes.c_float, ctypes.c_float, _I, _I,
                                    _FP, _FP, _I, _FP]),
    "ssla_hip_model_head_row": (_I, [_VP, _FP, _FP]),
    "ssla_hip_head_row": (_I, [ctypes.c_char_p, _FP, _FP]),
    "ssla_hip_oeva_write": (_I, [ctypes.c_char_p, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                 ctypes.POINTER(ctypes.c_ulonglong), _FP]),
    "ssla_hip_oeva_header": (_I, [ctypes.c_char_p, _UP]),
    "ssla_hip_oeva_read": (_I, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_ulonglong), _FP,
                                ctypes.c_uint]),
    "ssla_hip_oeva_diff": (_I, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_double,
                                ctypes.POINTER(abi.SslaHipOevaDiff)]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


class SslaHipError(RuntimeError):
    pass


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load (once) and type the library.  Raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise SslaHipError(f"{p} is not built; run `make -C {PKG_ROOT}` or "
                           "__graft_entry__.build()")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(rc: int, what: str = "") -> int:
    if rc < 0:
        msg = load().ssla_hip_last_error().decode(errors="replace")
        raise SslaHipError(f"{what or 'ssla_hip'} failed ({rc}): {msg}")
    return rc


def layout() -> dict:
    out = (ctypes.c_longlong * 7)()
    check(load().ssla_hip_abi_layout(out, 7), "abi_layout")
    keys = ("HybridInputRec", "HybridS2S3Config", "preds_offset",
            "HybridS2S3OutputSlot", "GpuTimingSlot", "HybridStrip", "LayerWeightsS2S3")
    return dict(zip(keys, list(out)))


def check_layout() -> None:
    got = layout()
    want = {
        "HybridInputRec": abi.INPUT_DTYPE.itemsize,
        "HybridS2S3Config": ctypes.sizeof(abi.HybridS2S3Config),
        "preds_offset": abi.HybridS2S3Config.preds.offset,
        "HybridS2S3OutputSlot": abi.OUTPUT_DTYPE.itemsize,
        "GpuTimingSlot": abi.TIMING_DTYPE.itemsize,
        "HybridStrip": ctypes.sizeof(abi.HybridStrip),
        "LayerWeightsS2S3": ctypes.sizeof(abi.LayerWeightsS2S3),
    }
    if got != want:
        raise SslaHipError(f"ABI layout mismatch: library {got} vs mirror {want}")
