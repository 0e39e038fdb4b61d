"""ctypes front end of oracle/cpu_attention.cpp — TEST INFRASTRUCTURE ONLY.

``decode_f64`` is the fast, threaded float64 restatement of the reference's
portable decode path (portable.py:155-205, batches.py:228-246), used to check
full-size configurations; ``decode_f32`` is the same path in float32, as the
reference computes it, which bench.py times as the CPU baseline;
``decode_splitk`` is the float32 restatement of the Metal split-K kernel
(metal_kernels.py:18-124), timed beside it. All three are pinned against
paged_attention.py (tests/test_oracle.py).
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_float, c_int, c_int64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY_PATH = HERE / "lib" / "libpda_oracle.so"

_lib = None


def library():
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.exists():
            raise FileNotFoundError(f"{LIBRARY_PATH} is not built; run `make -C {HERE}`")
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        lib.oracle_decode_f64.restype = None
        lib.oracle_decode_f64.argtypes = [c_void_p] * 6 + [c_int] * 6 + [
            c_int64, c_double, c_int, c_double, c_int]
        lib.oracle_decode_f32.restype = None
        lib.oracle_decode_f32.argtypes = [c_void_p] * 6 + [c_int] * 6 + [
            c_int64, c_float, c_int, c_float, c_int]
        lib.oracle_decode_splitk.restype = None
        lib.oracle_decode_splitk.argtypes = [c_void_p] * 6 + [c_int] * 6 + [
            c_int64, c_float, c_int, c_float, c_int, c_int]
        lib.oracle_half_to_float.argtypes = [c_void_p, c_void_p, c_int64]
        lib.oracle_float_to_half.argtypes = [c_void_p, c_void_p, c_int64]
        _lib = lib
    return _lib


def host_cores() -> int:
    return len(os.sched_getaffinity(0))


def _args(q, keys, values, tables, lengths):
    q = np.ascontiguousarray(q, dtype=np.float16)
    keys = np.ascontiguousarray(keys, dtype=np.float16)
    values = np.ascontiguousarray(values, dtype=np.float16)
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    return q, keys, values, tables, lengths


def decode_f64(q, keys, values, tables, lengths, *, page_size, scale, window=0,
               softcap=0.0, threads=None) -> np.ndarray:
    """Float64 portable-path oracle; returns ``[B, HQ, D]`` float64."""
    q, keys, values, tables, lengths = _args(q, keys, values, tables, lengths)
    batch, hq, dim = q.shape
    hkv = keys.shape[1]
    if hq % hkv:
        raise ValueError("query heads must be a multiple of kv heads")
    out = np.zeros((batch, hq, dim), dtype=np.float64)
    library().oracle_decode_f64(
        q.ctypes.data, keys.ctypes.data, values.ctypes.data, tables.ctypes.data,
        lengths.ctypes.data, out.ctypes.data, batch, hq, hkv, dim, page_size,
        tables.shape[1], keys.shape[0], scale, window, softcap,
        threads or host_cores())
    return out


def decode_f32(q, keys, values, tables, lengths, *, page_size, scale, window=0,
               softcap=0.0, threads=None) -> np.ndarray:
    """Float32 restatement of the portable path (gather, then dense
    attention in float32, portable.py:155-205); ``[B, HQ, D]`` fp16."""
    q, keys, values, tables, lengths = _args(q, keys, values, tables, lengths)
    batch, hq, dim = q.shape
    hkv = keys.shape[1]
    if hq % hkv:
        raise ValueError("query heads must be a multiple of kv heads")
    out = np.zeros((batch, hq, dim), dtype=np.float16)
    library().oracle_decode_f32(
        q.ctypes.data, keys.ctypes.data, values.ctypes.data, tables.ctypes.data,
        lengths.ctypes.data, out.ctypes.data, batch, hq, hkv, dim, page_size,
        tables.shape[1], keys.shape[0], scale, window, softcap,
        threads or host_cores())
    return out


def decode_splitk(q, keys, values, tables, lengths, *, page_size, scale, window=0,
                  softcap=0.0, splits=0, threads=None) -> np.ndarray:
    """Float32 split-K restatement of the Metal kernel; ``[B, HQ, D]`` fp16."""
    q, keys, values, tables, lengths = _args(q, keys, values, tables, lengths)
    batch, hq, dim = q.shape
    hkv = keys.shape[1]
    if hq % hkv:
        raise ValueError("query heads must be a multiple of kv heads")
    out = np.zeros((batch, hq, dim), dtype=np.float16)
    library().oracle_decode_splitk(
        q.ctypes.data, keys.ctypes.data, values.ctypes.data, tables.ctypes.data,
        lengths.ctypes.data, out.ctypes.data, batch, hq, hkv, dim, page_size,
        tables.shape[1], keys.shape[0], scale, window, softcap, splits,
        threads or host_cores())
    return out
