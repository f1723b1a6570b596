"""ctypes loader of oracle/attention_oracle.c -- TEST INFRASTRUCTURE ONLY.

Builds ``oracle/_build/libattn_oracle.so`` with ``make -C oracle`` on first
use when it is missing.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libattn_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        f64p = ctypes.POINTER(ctypes.c_double)
        f32p = ctypes.POINTER(ctypes.c_float)
        i = ctypes.c_int
        lib.oracle_attention_ld.argtypes = [u16p, u16p, u16p, f64p, f64p, i, i, i, i, i,
                                            ctypes.c_double, i]
        lib.oracle_attention_ld.restype = None
        lib.oracle_online_f32.argtypes = [u16p, u16p, u16p, f32p, i, i, i, i, i,
                                          ctypes.c_float, i, i, i]
        lib.oracle_online_f32.restype = None
        lib.oracle_rand_stream.argtypes = [ctypes.c_uint, i, ctypes.c_float, f32p]
        lib.oracle_rand_stream.restype = None
        lib.oracle_tile_softmax.argtypes = [f32p, f64p, f64p, f64p, i, i, ctypes.c_double, i]
        lib.oracle_tile_softmax.restype = None
        _lib = lib
    return _lib


def _u16(a: np.ndarray):
    a = np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def attention_ld(Q, K, V, causal=False, scale=None):
    """Long-double two-pass attention; returns (O float64, LSE float64)."""
    lib = _load()
    B, Hq, N, D = Q.shape
    Hkv = K.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    q, qp = _u16(Q)
    k, kp = _u16(K)
    v, vp = _u16(V)
    o = np.zeros((B, Hq, N, D), dtype=np.float64)
    lse = np.zeros((B, Hq, N), dtype=np.float64)
    lib.oracle_attention_ld(qp, kp, vp, o.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                            lse.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                            B, Hq, Hkv, N, D, float(scale), int(bool(causal)))
    return o, lse


def online_f32(Q, K, V, causal=False, scale=None, tile=32, round_p=False):
    """fp32 tiled online softmax in the reference scalar kernel's order."""
    lib = _load()
    B, Hq, N, D = Q.shape
    Hkv = K.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    q, qp = _u16(Q)
    k, kp = _u16(K)
    v, vp = _u16(V)
    o = np.zeros((B, Hq, N, D), dtype=np.float32)
    lib.oracle_online_f32(qp, kp, vp, o.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                          B, Hq, Hkv, N, D, float(scale), int(bool(causal)), int(tile),
                          int(bool(round_p)))
    return o


def rand_stream(seed: int, n: int, span: float) -> np.ndarray:
    """glibc srand(seed); (rand()/RAND_MAX - 0.5) * span for n draws."""
    lib = _load()
    out = np.zeros(n, dtype=np.float32)
    lib.oracle_rand_stream(seed, n, float(span), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def tile_softmax(x: np.ndarray, scale: float, normalize: bool):
    """Row softmax of a [rows, cols] fp32 tile in double; returns (out, max, sum)."""
    lib = _load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.zeros((rows, cols), dtype=np.float64)
    mx = np.zeros(rows, dtype=np.float64)
    sm = np.zeros(rows, dtype=np.float64)
    f64p = ctypes.POINTER(ctypes.c_double)
    lib.oracle_tile_softmax(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                            out.ctypes.data_as(f64p), mx.ctypes.data_as(f64p),
                            sm.ctypes.data_as(f64p), rows, cols, float(scale), int(normalize))
    return out, mx, sm
