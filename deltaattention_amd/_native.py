"""ctypes binding of libdeltaattn.so (the C ABI declared in include/deltaattn.h).

There is no fallback: if the library is missing or fails to load, every operation
raises ``NativeLibraryError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdeltaattn.so")

DA_BF16 = 1
DA_F16 = 2
DA_I32 = 3
DA_F32 = 4
DA_VARIANT = {"hybrid": 0, "sanity": 1, "pure_phase1": 2}
DA_SELECT_COSINE = 1
DA_SELECT_ARITH16 = 2
DA_NUM_STRIDES = 24

# (name, restype, argtypes) for every symbol of include/deltaattn.h
_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
SIGNATURES = {
    "da_last_error": (ctypes.c_char_p, []),
    "da_version": (_I, []),
    "da_select": (_I, [_P, _I, _L, _L, _L, _L, _L, _L, _L, _F, _I, _L, _L, _P, _P, _P]),
    "da_pack_workspace_size": (_L, [_L, _L, _L]),
    "da_pack": (_I, [_P, _P, _P, _I, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _P, _P, _P, _P,
                     _P, _P, _P, _L, _P]),
    "da_hybrid_workspace_size": (_L, [_L, _L, _L]),
    "da_hybrid_prefill": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _L, _L, _L, _L, _L, _L, _P,
                               _L, _P, _L, _F, _I, _I, _P, _L, _P]),
    "da_dense_prefill": (_I, [_P, _P, _P, _P, _I, _L, _L, _L, _L, _L, _L, _P, _I, _F, _P]),
    "da_select_varlen": (_I, [_P, _I, _L, _L, _L, _L, _L, _L, _P, _L, _F, _I, _L, _L, _P, _P, _L, _P]),
    "da_pack_varlen_workspace_size": (_L, [_L, _L, _L]),
    "da_pack_varlen": (_I, [_P, _P, _P, _I, _L, _L, _L, _L, _L, _L, _L, _L, _P, _L, _P, _P, _P, _P,
                            _P, _P, _P, _L, _P]),
    "da_hybrid_varlen_workspace_size": (_L, [_L, _L, _L]),
    "da_hybrid_prefill_varlen": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _L, _L, _L, _L, _L,
                                      _P, _P, _L, _P, _L, _F, _I, _I, _P, _L, _P]),
    "da_dense_prefill_varlen": (_I, [_P, _P, _P, _P, _I, _L, _L, _L, _L, _L, _P, _P, _L, _I, _F,
                                     _P]),
    "da_decode_update": (_I, [_P, _P, _I, _L, _L, _L, _L, _L, _P, _P, _L, _L, _L, _P, _P, _L, _L,
                              _L, _P, _P, _L, _L, _P, _L, _L, _L, _L, _F, _I, _P]),
    "da_decode_workspace_size": (_L, [_L, _L, _L, _L]),
    "da_decode_attention": (_I, [_P, _I, _L, _L, _L, _L, _L, _L, _P, _P, _L, _L, _L, _P, _L, _L,
                                 _P, _L, _P, _P, _L, _L, _L, _L, _L, _F, _P, _L, _L, _P, _L, _P]),
    "da_decode_attention_noalloc": (_I, [_P, _I, _L, _L, _L, _L, _L, _L, _P, _P, _L, _L, _L, _P, _L,
                                         _L, _P, _L, _P, _P, _L, _L, _L, _L, _L, _F, _P, _L, _L,
                                         _P]),
    "da_decode_step": (_I, [_P, _P]),
}


class DecodeStep(ctypes.Structure):
    """struct DaDecodeStep of include/deltaattn.h (field for field)."""
    _fields_ = [
        ("new_k", _P), ("new_v", _P), ("sn_b", _L), ("sn_h", _L),
        ("q", _P), ("sq_b", _L), ("sq_h", _L),
        ("out", _P), ("so_b", _L), ("so_h", _L),
        ("k_exact", _P), ("v_exact", _P), ("sx_b", _L), ("sx_h", _L), ("sx_s", _L),
        ("k_packed", _P), ("v_packed", _P), ("sp_b", _L), ("sp_h", _L), ("sp_s", _L),
        ("counts", _P), ("timestamps", _P), ("sc_b", _L), ("sc_h", _L),
        ("lengths", _P), ("capacity", _L),
        ("exact_seq_len", _L), ("total_seq_len", _L), ("window", _L),
        ("threshold", _F), ("use_cosine", ctypes.c_int32), ("scale", _F), ("dtype", ctypes.c_int32),
        ("B", _L), ("Hq", _L), ("Hkv", _L), ("D", _L),
        ("workspace", _P), ("workspace_bytes", _L),
    ]

DA_DECODE_SCRATCH_BYTES = 32 << 20


class NativeLibraryError(RuntimeError):
    """libdeltaattn.so is missing or could not be loaded."""


class DeltaAttnError(RuntimeError):
    """A C-ABI call returned an error status."""

    def __init__(self, what: str, code: int, message: str):
        super().__init__(f"{what} failed ({code}): {message}")
        self.code = code


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """Load libdeltaattn.so once; raise NativeLibraryError if it is not there."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryError(
                    f"{LIB_PATH} is not built; run `python -m deltaattention_amd.build` "
                    "(there is no non-native fallback)")
            try:
                handle = ctypes.CDLL(LIB_PATH)
            except OSError as e:
                raise NativeLibraryError(f"cannot load {LIB_PATH}: {e}") from e
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().da_last_error()
        raise DeltaAttnError(what, rc, msg.decode() if msg else "")


def strides_array(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * DA_NUM_STRIDES)()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr


def dtype_code(*ts) -> int:
    """DA_BF16, DA_F16 or DA_F32 for tensors that all share one of those dtypes (the entry
    points that do not take fp32, the decode ones, refuse DA_F32 with DA_ERR_UNSUPPORTED)."""
    import torch
    codes = {torch.bfloat16: DA_BF16, torch.float16: DA_F16, torch.float32: DA_F32}
    dt = ts[0].dtype
    if dt not in codes:
        raise TypeError(f"expected bfloat16, float16 or float32 tensors, got {dt}")
    for t in ts[1:]:
        if t is not None and t.dtype != dt:
            raise TypeError(f"all tensors must share one dtype ({dt}), got {t.dtype}")
    return codes[dt]
