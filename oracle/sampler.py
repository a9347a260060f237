"""ctypes wrapper of the C sampler restatement (TEST INFRASTRUCTURE ONLY)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from .build_oracle import OUT, build

_lib = None


def _L():
    global _lib
    if _lib is None:
        if not OUT.exists():
            build()
        _lib = C.CDLL(str(OUT))
        _lib.oracle_sample.restype = None
        _lib.oracle_sample.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int] + [C.c_void_p] * 5 + [C.c_int, C.c_void_p]
        _lib.oracle_probs_row.restype = None
        _lib.oracle_probs_row.argtypes = [C.c_void_p, C.c_int, C.c_float, C.c_float, C.c_int, C.c_float, C.c_int, C.c_void_p]
        _lib.oracle_exp2.restype = C.c_float
        _lib.oracle_exp2.argtypes = [C.c_float]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def sample(logits_bits: np.ndarray, temps, top_ps, top_ks, min_ps, uniforms, flags: int) -> np.ndarray:
    """logits_bits: uint16 [B, V] raw bf16; returns int64 ids [B]."""
    lb = np.ascontiguousarray(logits_bits, dtype=np.uint16)
    b, v = lb.shape
    f = lambda a, dt: None if a is None else np.ascontiguousarray(a, dtype=dt)
    t, p, k, m, u = f(temps, np.float32), f(top_ps, np.float32), f(top_ks, np.int32), f(min_ps, np.float32), f(uniforms, np.float32)
    out = np.zeros(b, dtype=np.int64)
    _L().oracle_sample(lb.ctypes.data, v, b, v, _p(t), _p(p), _p(k), _p(m), _p(u), int(flags), out.ctypes.data)
    return out


def exp2(x: float) -> float:
    return _L().oracle_exp2(float(x))


def probs(logits_bits_row: np.ndarray, temp: float, top_p: float, top_k: int, min_p: float, flags: int) -> np.ndarray:
    """Per-id probability of one row under the explicit-draw sampler."""
    lb = np.ascontiguousarray(logits_bits_row, dtype=np.uint16)
    out = np.zeros(lb.shape[0], dtype=np.float64)
    _L().oracle_probs_row(lb.ctypes.data, lb.shape[0], temp, top_p, int(top_k), min_p, int(flags), out.ctypes.data)
    return out
