"""ctypes binding to the C restatement of ``cpu_attn`` (oracle/cpu_attn.c).

Test infrastructure only.  Builds ``oracle/_build/libkf_oracle.so`` with make
on first use if it is not there.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libkf_oracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        for name, ct in (("kf_oracle_attn_f32", ctypes.c_float), ("kf_oracle_attn_f64", ctypes.c_double)):
            fn = getattr(_lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 6
        _lib.kf_oracle_half_to_float.restype = ctypes.c_float
        _lib.kf_oracle_half_to_float.argtypes = [ctypes.c_ushort]
        _lib.kf_oracle_float_to_half.restype = ctypes.c_ushort
        _lib.kf_oracle_float_to_half.argtypes = [ctypes.c_float]
    return _lib


def cpu_attn(Q, K, V, dtype=np.float64):
    """Brute-force attention of cpu_attn.c; returns (O, Mi, Li) in ``dtype``."""
    B, H_q, q_len, D = Q.shape
    _, H_kv, kv_len, _ = K.shape
    q = np.ascontiguousarray(Q, dtype=dtype)
    k = np.ascontiguousarray(K, dtype=dtype)
    v = np.ascontiguousarray(V, dtype=dtype)
    O = np.empty((B, H_q, q_len, D), dtype=dtype)
    M = np.empty((B, H_q, q_len), dtype=dtype)
    L = np.empty((B, H_q, q_len), dtype=dtype)
    fn = lib().kf_oracle_attn_f64 if dtype == np.float64 else lib().kf_oracle_attn_f32
    rc = fn(q.ctypes.data, k.ctypes.data, v.ctypes.data, O.ctypes.data, M.ctypes.data,
            L.ctypes.data, B, q_len, kv_len, H_q, H_kv, D)
    if rc != 0:
        raise ValueError(f"kf_oracle_attn rejected the shape (rc={rc})")
    return O, M, L


def float_to_half_bits(x: float) -> int:
    return int(lib().kf_oracle_float_to_half(ctypes.c_float(x)))


def half_bits_to_float(h: int) -> float:
    return float(lib().kf_oracle_half_to_float(ctypes.c_ushort(h)))
