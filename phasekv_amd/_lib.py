"""ctypes binding of ``libphasekv_hip.so`` (the C ABI declared in include/phasekv_hip.h).

The library is required: there is no CPU or torch fallback.  If it is missing,
every entry point raises ``RuntimeError`` telling how to build it.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libphasekv_hip.so")

PK_OK = 0
PK_ERR_INVALID = -1
PK_ERR_RUNTIME = -2

PK_DTYPE_F16 = 0
PK_DTYPE_BF16 = 1
PK_DTYPE_F32 = 2

PK_SEG_KIVI = 0
PK_SEG_TOKEN = 1
PK_SEG_FP16 = 2

PK_MAX_SEGMENTS_PER_LAUNCH = 8
PK_NOALLOC_SCRATCH_BYTES = 16 << 20
PK_MAX_PARTIAL_SETS = 4
PK_FLAG_GENERIC_KERNEL = 1
PK_FLAG_REQUIRE_MFMA = 2

PK_META_CHANNEL_MAJOR = 0
PK_META_GROUP_MAJOR = 1
PK_CODES_CHANNEL_MAJOR = 0
PK_CODES_TOKEN_MAJOR = 1
PK_LAYOUT_META_TRANSPOSED = 1
PK_LAYOUT_CODES_TRANSPOSED = 2

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p


class PkSegment(ctypes.Structure):
    """Mirror of ``pk_segment``."""

    _fields_ = [
        ("kind", _c_i32), ("length", _c_i32), ("k_bits", _c_i32), ("v_bits", _c_i32),
        ("k_group", _c_i32), ("v_group", _c_i32), ("splits", _c_i32), ("split_len", _c_i32),
        ("k_meta_layout", _c_i32), ("k_data_layout", _c_i32),
        ("seq_lens", _c_vp),
        ("k_data", _c_vp), ("k_scale", _c_vp), ("k_mins", _c_vp),
        ("v_data", _c_vp), ("v_scale", _c_vp), ("v_mins", _c_vp),
        ("k_data_bstride", _c_i64), ("k_data_hstride", _c_i64),
        ("k_meta_bstride", _c_i64), ("k_meta_hstride", _c_i64),
        ("v_data_bstride", _c_i64), ("v_data_hstride", _c_i64),
        ("v_meta_bstride", _c_i64), ("v_meta_hstride", _c_i64),
        ("tok_stride", _c_i64),
    ]


class PkDecodeProblem(ctypes.Structure):
    """Mirror of ``pk_decode_problem``."""

    _fields_ = [
        ("batch", _c_i32), ("num_q_heads", _c_i32), ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("q", _c_vp), ("q_bstride", _c_i64), ("q_hstride", _c_i64),
        ("segments", ctypes.POINTER(PkSegment)), ("num_segments", _c_i32),
        ("flags", _c_i32),
        ("table", _c_vp), ("table_count", _c_i32), ("table_bits", _c_i32),
    ]



class PkPartialSet(ctypes.Structure):
    """Mirror of ``pk_partial_set``."""

    _fields_ = [
        ("m", _c_vp), ("l", _c_vp), ("acc", _c_vp), ("rows", _c_i64), ("n", _c_i32),
        ("pad_", _c_i32), ("outer_stride", _c_i64), ("inner_stride", _c_i64),
    ]

# name -> (restype, argtypes)
_SIGNATURES = {
    "pk_last_error": (ctypes.c_char_p, []),
    "pk_version": (ctypes.c_char_p, []),
    "pk_device_info": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                      ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                      ctypes.POINTER(ctypes.c_int)]),
    "pk_pack_low_bits": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, ctypes.c_int, _c_vp, _c_vp]),
    "pk_unpack_low_bits": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, ctypes.c_int, _c_i64, _c_vp,
                                          _c_vp]),
    "pk_quantize_pack": (ctypes.c_int, [_c_vp, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64),
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        _c_vp, _c_vp, _c_vp, ctypes.c_int, _c_vp]),
    "pk_quantize_pack_kv": (ctypes.c_int, [_c_vp, _c_vp, ctypes.c_int, ctypes.c_int, _c_i64,
                                           ctypes.c_int, ctypes.c_int, _c_vp, _c_vp, _c_vp, _c_vp,
                                           _c_vp, _c_vp, _c_vp]),
    "pk_unpack_dequantize": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, ctypes.c_int,
                                            ctypes.POINTER(_c_i64), ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _c_i64, _c_vp, _c_vp]),
    "pk_decode_workspace_size": (ctypes.c_int, [ctypes.POINTER(PkDecodeProblem),
                                                ctypes.POINTER(ctypes.c_size_t),
                                                ctypes.POINTER(_c_i32)]),
    "pk_segment_table_entry_bytes": (ctypes.c_size_t, []),
    "pk_segment_table_write": (ctypes.c_int, [_c_vp, _c_i32, _c_i32, ctypes.POINTER(PkSegment),
                                              _c_i32, _c_vp]),
    "pk_decode_partials": (ctypes.c_int, [ctypes.POINTER(PkDecodeProblem), _c_vp,
                                          ctypes.c_size_t, _c_vp]),
    "pk_decode_combine": (ctypes.c_int, [ctypes.POINTER(PkDecodeProblem), _c_vp, _c_vp, _c_vp,
                                         _c_vp, _c_vp, _c_vp]),
    "pk_fused_decode": (ctypes.c_int, [ctypes.POINTER(PkDecodeProblem), _c_vp, ctypes.c_size_t,
                                       _c_vp, _c_vp]),
    "pk_fused_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(PkDecodeProblem), _c_vp, _c_vp]),
    "pk_merge_partials": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_i32, _c_vp,
                                         _c_vp, _c_vp, _c_vp, _c_vp]),
    "pk_merge_partial_sets": (ctypes.c_int, [ctypes.POINTER(PkPartialSet), _c_i32, _c_i64,
                                             _c_i64, _c_i32, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "pk_append_hot": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp,
                                     _c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, _c_i64, _c_i64, _c_vp]),
    "pk_append_hot_rows": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                          _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_i64,
                                          _c_i64, _c_i64, _c_vp]),
    "pk_rope_append_hot": (ctypes.c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp,
                                          _c_i64, ctypes.c_int, _c_vp, _c_vp, _c_vp, _c_i64,
                                          _c_i64, _c_i64,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          _c_i64, _c_i64, _c_vp]),
    "pk_cool_hot": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_vp,
                                   _c_vp, _c_vp, _c_vp]),
    "pk_cool_pack_supported": (ctypes.c_int, [_c_i64, ctypes.c_int, _c_i64, _c_i64,
                                              ctypes.c_int]),
    "pk_cool_pack_hot": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, _c_i64, _c_i64, _c_i64,
                                        ctypes.c_int, ctypes.c_int, _c_vp, _c_vp, _c_vp, _c_vp,
                                        _c_vp, _c_vp, _c_vp, _c_vp]),
    "pk_prompt_votes": (ctypes.c_int, [_c_vp, ctypes.c_int, _c_i64, _c_i64, _c_i64, _c_i64,
                                       ctypes.POINTER(_c_i64), ctypes.c_int, ctypes.c_int, _c_vp,
                                       _c_vp]),
    "pk_select_prompt": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                        ctypes.c_int, ctypes.c_int, _c_vp, _c_vp]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load and return the shared library (raises RuntimeError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m phasekv_amd.build` "
                "(there is no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    """Map a C status to the reference's exception types."""
    if rc == PK_OK:
        return
    msg = load().pk_last_error().decode("utf-8", "replace")
    if rc == PK_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def require_device(*tensors) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(
                f"phasekv_amd runs on a ROCm GPU; got a tensor on {t.device} "
                "(there is no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def i64_array(values):
    arr = (_c_i64 * len(values))(*[int(v) for v in values])
    return arr


def device_cu_count(device: torch.device) -> int:
    lib = load()
    cus = ctypes.c_int(0)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    check(lib.pk_device_info(idx, ctypes.byref(cus), None, None, None), "pk_device_info")
    return cus.value
