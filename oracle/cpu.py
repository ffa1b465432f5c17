"""ctypes wrapper of the C oracle restatement (oracle/libexl3cpu.so) -- TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, the smoke entry point and bench.py's cpu_baseline leg.
Arrays are numpy; fp16 data is passed as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libexl3cpu.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE, "libexl3cpu.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        p, i, i64 = C.c_void_p, C.c_int, C.c_int64
        L.exl3cpu_reconstruct.argtypes = [p, i, i, i, i, p, i]
        L.exl3cpu_linear.argtypes = [p, i, i, i, p, i, i, p, p, p, i]
        L.exl3cpu_had_in.argtypes = [p, i, i, p, p]
        L.exl3cpu_had_out.argtypes = [p, i, i, p, p]
        L.exl3cpu_decode_states.argtypes = [p, i64, i, p]
        L.exl3cpu_f64_to_f16.argtypes = [C.c_double]
        L.exl3cpu_f64_to_f16.restype = C.c_uint16
        L.exl3cpu_max_threads.restype = i
        _lib = L
    return _lib


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    assert a.dtype in (np.uint16, np.int16), a.dtype
    return a.view(np.uint16)


def _ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


def max_threads() -> int:
    return int(lib().exl3cpu_max_threads())


def reconstruct(trellis, bits: int, cb: int, threads: int = 0) -> np.ndarray:
    tr = _u16(trellis)
    k, n = tr.shape[0] * 16, tr.shape[1] * 16
    W = np.empty((k, n), dtype=np.uint16)
    rc = lib().exl3cpu_reconstruct(_ptr(tr), k, n, bits, cb, _ptr(W), threads)
    assert rc == 0, rc
    return W.view(np.float16)


def linear(x, trellis, bits: int, suh, svh, cb: int, threads: int = 0) -> np.ndarray:
    """Faithful EXL3 linear, fp16 result [m, n]."""
    tr = _u16(trellis)
    xx = _u16(np.atleast_2d(np.asarray(x, dtype=np.float16)))
    m, k = xx.shape
    n = tr.shape[1] * 16
    su = _u16(np.asarray(suh, dtype=np.float16))
    sv = _u16(np.asarray(svh, dtype=np.float16))
    y = np.empty((m, n), dtype=np.uint16)
    rc = lib().exl3cpu_linear(_ptr(xx), m, k, n, _ptr(tr), bits, cb, _ptr(su), _ptr(sv), _ptr(y), threads)
    assert rc == 0, rc
    return y.view(np.float16)


def had_in(x, suh) -> np.ndarray:
    xx = _u16(np.atleast_2d(np.asarray(x, dtype=np.float16)))
    su = _u16(np.asarray(suh, dtype=np.float16))
    out = np.empty_like(xx)
    assert lib().exl3cpu_had_in(_ptr(xx), xx.shape[0], xx.shape[1], _ptr(su), _ptr(out)) == 0
    return out.view(np.float16)


def had_out(c, svh) -> np.ndarray:
    cc = _u16(np.atleast_2d(np.asarray(c, dtype=np.float16)))
    sv = _u16(np.asarray(svh, dtype=np.float16))
    out = np.empty_like(cc)
    assert lib().exl3cpu_had_out(_ptr(cc), cc.shape[0], cc.shape[1], _ptr(sv), _ptr(out)) == 0
    return out.view(np.float16)


def decode_states(states, cb: int) -> np.ndarray:
    st = _u16(states)
    out = np.empty_like(st)
    assert lib().exl3cpu_decode_states(_ptr(st), st.size, cb, _ptr(out)) == 0
    return out.view(np.float16)


def f64_to_f16_bits(v: float) -> int:
    return int(lib().exl3cpu_f64_to_f16(float(v)))
