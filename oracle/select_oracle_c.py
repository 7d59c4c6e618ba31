"""ctypes binding of oracle/select_oracle.c -- TEST INFRASTRUCTURE ONLY.

Same contract as ``delta_oracle.select_delta`` (tritonModules.py:7-69), computed by the
C restatement so that sequence lengths of 32K-128K finish in about a second.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Tuple

import numpy as np

from .delta_oracle import chunking, select_threshold

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_select.so")
_lib = None


def build() -> str:
    """Compile the C restatement with oracle/Makefile; returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_select_delta.restype = ctypes.c_int
        lib.oracle_select_delta.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_float, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_void_p]
        _lib = lib
    return _lib


ARITH = {"fp32": 0, "bf16": 1, "fp16": 2}


def select_delta(k: np.ndarray, threshold: float, chunk_size: int = 512, divide_to: int = 0,
                 metric: str = "euclidean", arith: str = "fp32") -> Tuple[np.ndarray, np.ndarray]:
    """keep [B,H,N] int32, chunk_counts [B,H,nc] int32 (see delta_oracle.select_delta).

    ``arith`` "bf16" / "fp16" rounds every difference, square and tree addition of the
    Euclidean distance to that type (the reference's 16-bit Triton arithmetic,
    tritonModules.py:55-58); "fp32" is the build's default definition."""
    k32 = np.ascontiguousarray(k, dtype=np.float32)
    B, H, N, D = k32.shape
    cs, nc = chunking(N, chunk_size, divide_to)
    thr = select_threshold(threshold, metric)
    keep = np.zeros((B, H, N), dtype=np.int32)
    counts = np.zeros((B, H, nc), dtype=np.int32)
    rc = _load().oracle_select_delta(
        k32.ctypes.data, B, H, N, D, ctypes.c_float(float(thr)), cs, nc,
        1 if metric == "cosine" else 0, ARITH[arith], keep.ctypes.data, counts.ctypes.data)
    if rc != 0:
        raise ValueError(f"oracle_select_delta failed ({rc}) for head_dim {D}")
    return keep, counts
