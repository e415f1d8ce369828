"""GEMM oracles (test infrastructure only; see oracle/__init__.py).

Semantics restated from frisk.gemm: C = op(A).op(B) (clear_accum) or
C += op(A).op(B) (include/Dialect/Frisk/IR/FriskOps.td:252-292; the read of C
when not clearing: lib/Dialect/Frisk/IR/FriskOps.cpp:416-426 and
lib/Dialect/Frisk/Transforms/LegacyFragmentNormalization.cpp:503-513), with
m/k/n derived from the operand shapes as ffi/ir.cpp:335-337 does.
"""
from __future__ import annotations

import numpy as np


def effective(a: np.ndarray, trans: bool) -> np.ndarray:
    """op(X): X or X^T (transA/transB of ffi/ir.cpp:335-337)."""
    return a.T if trans else a


def gemm_fp64(a, b, *, trans_a=False, trans_b=False, c=None, clear_accum=True):
    """Textbook GEMM in float64 on the exactly decoded inputs.

    The north star's fp64 host oracle; C is read only when clear_accum is
    false (FriskOps.cpp:416-426)."""
    A = effective(np.asarray(a, dtype=np.float64), trans_a)
    B = effective(np.asarray(b, dtype=np.float64), trans_b)
    out = A @ B
    if not clear_accum:
        out = out + np.asarray(c, dtype=np.float64)
    return out


def gemm_fp32_rank1(a, b, *, trans_a=False, trans_b=False):
    """The reference's fp32 oracle order: a sequence of K rank-1 updates, each
    product and each sum rounded to fp32 (run_execution.py:58-63:
    `s = float32(s + float32(q[:, t, None] * k[None, :, t]))`)."""
    A = effective(np.asarray(a, dtype=np.float32), trans_a)
    B = effective(np.asarray(b, dtype=np.float32), trans_b)
    m, k = A.shape
    n = B.shape[1]
    s = np.zeros((m, n), dtype=np.float32)
    for t in range(k):
        s = np.float32(s + np.float32(A[:, t, None] * B[None, t, :]))
    return s


def gemm_int(a, b, *, trans_a=False, trans_b=False):
    """Exact integer GEMM (int8 x int8 -> int64; the int32 result is exact
    while |sum| < 2^31)."""
    A = effective(np.asarray(a, dtype=np.int64), trans_a)
    B = effective(np.asarray(b, dtype=np.int64), trans_b)
    return A @ B


def e4m3fn_decode_table() -> np.ndarray:
    """float64 value of every OCP FP8 E4M3FN byte (1 sign, 4 exponent bits
    with bias 7, 3 mantissa bits; exponent 0 is subnormal m/8 * 2^-6; the
    pattern S.1111.111 is NaN; there are no infinities)."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            out[code] = np.nan
        elif e == 0:
            out[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            out[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


_E4M3 = e4m3fn_decode_table()


def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """Decode an array of e4m3fn bytes (uint8) to float64."""
    return _E4M3[np.asarray(codes, dtype=np.uint8)]


def bf16_decode(bits: np.ndarray) -> np.ndarray:
    """Decode bf16 bit patterns (uint16) to float64 (bf16 is the top half of
    an IEEE binary32)."""
    u = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return u.view(np.float32).astype(np.float64)


def row_scaled_error(got, ref) -> float:
    """max_i max_j |got - ref| / max_j |ref| (the north star's
    |err| <= tol * ||row||_inf criterion, as one ratio)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref).max(axis=-1)
    rown = np.abs(ref).max(axis=-1)
    rown = np.where(rown == 0, 1.0, rown)
    return float((err / rown).max())
