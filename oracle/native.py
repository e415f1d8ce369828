"""ctypes access to oracle/liboracle.so (test infrastructure only)."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        i64, dp, c_int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
        lib.oracle_gemm_f64.argtypes = [i64, i64, i64, dp, i64, c_int, dp, i64, c_int, dp, i64, c_int]
        lib.oracle_gemm_f64.restype = c_int
        lib.oracle_attn_f64.argtypes = [i64, i64, i64, dp, dp, dp, c_int, ctypes.c_double, dp, dp,
                                        c_int]
        lib.oracle_attn_f64.restype = c_int
        lib.oracle_attn_rows_f64.argtypes = [i64, i64, i64, dp, i64, dp, dp, dp, c_int,
                                             ctypes.c_double, dp, dp, c_int]
        lib.oracle_attn_rows_f64.restype = c_int
        lib.oracle_max_threads.restype = c_int
        _lib = lib
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def gemm_f64(a, b, *, trans_a=False, trans_b=False, threads=0):
    a = np.ascontiguousarray(a, dtype=np.float64)
    b = np.ascontiguousarray(b, dtype=np.float64)
    m = a.shape[1] if trans_a else a.shape[0]
    k = a.shape[0] if trans_a else a.shape[1]
    n = b.shape[0] if trans_b else b.shape[1]
    c = np.empty((m, n), dtype=np.float64)
    rc = load().oracle_gemm_f64(m, n, k, _p(a), a.shape[1], int(trans_a), _p(b), b.shape[1],
                                int(trans_b), _p(c), n, threads)
    assert rc == 0
    return c


def attn_f64(q, k, v, *, causal=False, scale=None, threads=0):
    """One head: q [sq, d], k/v [sk, d] -> (o [sq, d], lse [sq])."""
    q = np.ascontiguousarray(q, dtype=np.float64)
    k = np.ascontiguousarray(k, dtype=np.float64)
    v = np.ascontiguousarray(v, dtype=np.float64)
    sq, d = q.shape
    sk = k.shape[0]
    if scale is None:
        scale = d ** -0.5
    o = np.empty((sq, d))
    lse = np.empty(sq)
    rc = load().oracle_attn_f64(sq, sk, d, _p(q), _p(k), _p(v), int(causal), float(scale), _p(o),
                                _p(lse), threads)
    assert rc == 0
    return o, lse


def attn_rows_f64(q, k, v, rows, *, causal=False, scale=None, threads=0):
    """Rows `rows` of one head: q [sq, d] (all rows), k/v [sk, d] ->
    (o [len(rows), d], lse [len(rows)]); each row's causal mask follows its
    index in q."""
    q = np.ascontiguousarray(q, dtype=np.float64)
    k = np.ascontiguousarray(k, dtype=np.float64)
    v = np.ascontiguousarray(v, dtype=np.float64)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    sq, d = q.shape
    sk = k.shape[0]
    if scale is None:
        scale = d ** -0.5
    o = np.empty((len(rows), d))
    lse = np.empty(len(rows))
    rc = load().oracle_attn_rows_f64(sq, sk, d, _p(rows), len(rows), _p(q), _p(k), _p(v),
                                     int(causal), float(scale), _p(o), _p(lse), threads)
    assert rc == 0
    return o, lse


def max_threads() -> int:
    return int(load().oracle_max_threads())
