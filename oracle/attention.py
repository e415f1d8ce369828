"""Attention oracles (test infrastructure only; see oracle/__init__.py).

* attention_fp64 -- fp64 dots and a stable softmax, the high-precision path
  of benchmark/layout/execution/tail_attention_reference.py:81-85 and
  :88-114, generalised to any head_dim, a causal mask (the FA tile program
  of tmp/ir.mlir:89-157 has none; key j visible to query i iff
  j <= i + seq_k - seq_q) and the natural-log LSE.
* ordered_sum / strict_probability / fp64_probability / tile_oracle -- the
  reference's strict D64 oracle (tail_attention_reference.py:49-114): FP32
  balanced tree over modulo-8 lane subgroups, exp2(log2e * (s - max)), P
  rounded to f16 before the FP32/FP64 value product.
* fixture_inputs / analytical -- the reference's analytic fixtures
  (:125-200, :224-243) with their closed-form outputs.
* fixed_tile_reference / fixed_tile_cases -- the 64x16 fixed-ABI attention
  oracle and its 15 inputs (run_execution.py:58-68).
"""
from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------
# fp64 attention (BHSD), causal mask, LSE
# ----------------------------------------------------------------------------


def attention_fp64(q, k, v, *, causal=False, scale=None, chunk=256):
    """O[b,h,i] = sum_j softmax_j(scale * q_i.k_j) v_j in float64.

    Returns (O, LSE) with LSE = ln sum_j exp(scale * q_i.k_j) over visible
    keys; rows without a visible key give O = 0, LSE = -inf."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, h, sq, d = q.shape
    sk = k.shape[2]
    if scale is None:
        scale = d ** -0.5
    out = np.zeros((b, h, sq, d))
    lse = np.full((b, h, sq), -np.inf)
    diag = sk - sq
    for bi in range(b):
        for hi in range(h):
            kt = k[bi, hi].T
            for s0 in range(0, sq, chunk):
                s1 = min(sq, s0 + chunk)
                s = (q[bi, hi, s0:s1] @ kt) * scale
                if causal:
                    i = np.arange(s0, s1)[:, None]
                    j = np.arange(sk)[None, :]
                    s = np.where(j <= i + diag, s, -np.inf)
                m = s.max(axis=-1, keepdims=True)
                live = np.isfinite(m[:, 0])
                m = np.where(np.isfinite(m), m, 0.0)
                e = np.exp(s - m)
                den = e.sum(axis=-1, keepdims=True)
                with np.errstate(invalid="ignore", divide="ignore"):
                    o = (e @ v[bi, hi]) / den
                    lrow = np.log(den[:, 0]) + m[:, 0]
                out[bi, hi, s0:s1] = np.where(live[:, None], o, 0.0)
                lse[bi, hi, s0:s1] = np.where(live, lrow, -np.inf)
    return out, lse


# ----------------------------------------------------------------------------
# The reference's strict D64 tile oracle
# ----------------------------------------------------------------------------

D64 = 64
TILE = 64
SCORE_SCALE = np.float32(0.125)  # tail_attention_reference.py:14
LOG2_E = np.array(0x3FB8AA3B, dtype=np.uint32).view(np.float32)[()]  # :15
ERROR = dict(strict_atol=3e-5, strict_rtol=3e-4, fp64_atol=4e-5, fp64_rtol=4e-4)  # :19
EXACT = ("uniform-sparse-value", "last-key-dominant", "tail-uniform")


def ordered_sum(exponent: np.ndarray) -> np.ndarray:
    """FP32 sum of a row as the reference's kernel performs it
    (tail_attention_reference.py:49-71): lane l in 0..3 owns the column
    pairs (2l + 8i, 2l + 8i + 1); each lane's values are summed by a
    balanced binary tree padded with zeros to a power of two; the four lane
    sums combine as (l0 + l1) + (l2 + l3)."""
    x = np.asarray(exponent, dtype=np.float32)
    n = x.shape[-1]
    lanes = []
    for lane in range(4):
        cols = [c for c in range(n) if (c // 2) % 4 == lane]
        if not cols:
            lanes.append(np.zeros(x.shape[:-1], dtype=np.float32))
            continue
        width = 1 << (len(cols) - 1).bit_length()
        tree = np.zeros(x.shape[:-1] + (width,), dtype=np.float32)
        tree[..., : len(cols)] = x[..., cols]
        while tree.shape[-1] > 1:
            tree = np.add(tree[..., 0::2], tree[..., 1::2], dtype=np.float32)
        lanes.append(tree[..., 0])
    left = np.add(lanes[0], lanes[1], dtype=np.float32)
    right = np.add(lanes[2], lanes[3], dtype=np.float32)
    return np.add(left, right, dtype=np.float32)[..., None]


def strict_probability(dot: np.ndarray) -> np.ndarray:
    """f16 P from fp64 dots: fp32 scale, fp32 row max, exp2 of
    log2e * (s - max), ordered fp32 sum, fp32 division, f16 rounding
    (tail_attention_reference.py:74-79)."""
    score = np.multiply(dot.astype(np.float32), SCORE_SCALE, dtype=np.float32)
    centered = np.subtract(score, score.max(axis=-1, keepdims=True), dtype=np.float32)
    e = np.exp2(np.multiply(centered, LOG2_E, dtype=np.float32), dtype=np.float32)
    return np.divide(e, ordered_sum(e), dtype=np.float32).astype(np.float16)


def fp64_probability(dot: np.ndarray) -> np.ndarray:
    """f16 P from an fp64 stable softmax (tail_attention_reference.py:82-86)."""
    score = dot * np.float64(SCORE_SCALE)
    e = np.exp(score - score.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float16)


def tile_oracle(q, k, v, mode: str) -> np.ndarray:
    """The reference's D64 oracle (tail_attention_reference.py:88-114):
    fp64 dots, P from `mode` ('strict' | 'fp64'), then P.V with P in f16
    and V widened to fp64; output fp32 ('strict') or fp64."""
    kern = {"strict": strict_probability, "fp64": fp64_probability}[mode]
    out_t = {"strict": np.float32, "fp64": np.float64}[mode]
    b, h, n, d = q.shape
    out = np.empty(q.shape, dtype=out_t)
    with np.errstate(under="ignore"):
        for bi in range(b):
            for hi in range(h):
                dot = q[bi, hi].astype(np.float64) @ k[bi, hi].astype(np.float64).T
                p = kern(dot)
                out[bi, hi] = p.astype(np.float64) @ v[bi, hi].astype(np.float64)
    return out


def _tail_start(n: int) -> int:
    return ((n - 1) // TILE) * TILE


def _boundary_keys(n: int):
    return tuple(dict.fromkeys((0, min(TILE - 1, n - 1), min(TILE, n - 1),
                                max(0, _tail_start(n) - 1), _tail_start(n),
                                max(0, n - 2), n - 1)))


def _one_hot_values(v: np.ndarray, keys, dtype=np.float16) -> None:
    """One nonzero V per feature (tail_attention_reference.py:125-132)."""
    b, h, _, d = v.shape
    heads = (np.arange(b * h).reshape(b, h) % 512).astype(np.float32) / 512
    for feature in range(d):
        value = 0.125 + heads + (feature % 8) / 32
        v[..., keys[feature % len(keys)], feature] = value.astype(dtype)


def fixture_inputs(shape, name: str, dtype=np.float16):
    """The exact fixtures of tail_attention_reference.py:153-200 (EXACT
    names), for any (B, H, N, D) and element type."""
    b, h, n, d = shape
    q, k, v = (np.zeros(shape, dtype=dtype) for _ in range(3))
    if name == "tail-uniform":
        start = _tail_start(n)
        _one_hot_values(v, tuple(range(start, n)), dtype)
        q[..., :, 0] = 1
        k[..., :start, 0] = -8192
        k[..., start:, 0] = 8192
        return q, k, v
    keys = _boundary_keys(n)
    _one_hot_values(v, keys, dtype)
    if name == "last-key-dominant":
        q[..., :, 0] = 1
        if n > 1:
            q[..., -1, 0] = -1
            k[..., :-1, 0] = -8192
        k[..., -1, 0] = 8192
    elif name != "uniform-sparse-value":
        raise ValueError(name)
    return q, k, v


def analytical(v, name: str, *, fp64: bool, coefficient_dtype=np.float16):
    """Closed-form output of an exact fixture (tail_attention_reference.py:
    224-243): uniform weight 1/count rounded to the P type, times the single
    nonzero V of each feature."""
    v = np.asarray(v)
    n = v.shape[-2]
    dtype = np.float64 if fp64 else np.float32

    def coefficient(count):
        return np.float64(coefficient_dtype(dtype(1) / dtype(count)))

    result = np.empty(v.shape, dtype=dtype)
    if name == "uniform-sparse-value":
        result[...] = coefficient(n) * v.sum(axis=-2, dtype=np.float64, keepdims=True)
    elif name == "tail-uniform":
        result[...] = coefficient(n - _tail_start(n)) * v.sum(axis=-2, dtype=np.float64,
                                                              keepdims=True)
    elif n == 1:
        result[...] = v
    else:
        result[..., :-1, :] = v[..., -1:, :]
        result[..., -1, :] = coefficient(n - 1) * v[..., :-1, :].sum(axis=-2, dtype=np.float64)
    return result


# ----------------------------------------------------------------------------
# The 64x16 fixed-ABI attention tile (run_execution.py:58-68)
# ----------------------------------------------------------------------------


def fixed_tile_reference(q, k, v) -> np.ndarray:
    """fp32 rank-1 products for S (K = 16), scale 0.25, fp32 softmax, P
    rounded to f16, fp32 rank-1 products for P.V (run_execution.py:58-64)."""
    q, k, v = (np.asarray(x).astype(np.float32) for x in (q, k, v))
    s = np.zeros((64, 64), dtype=np.float32)
    for t in range(16):
        s = np.float32(s + np.float32(q[:, t, None] * k[None, :, t]))
    s = np.float32(s * np.float32(0.25))
    e = np.exp(np.float32(s - s.max(axis=1, keepdims=True)), dtype=np.float32)
    prob = np.float32(e / e.sum(axis=1, keepdims=True, dtype=np.float32))
    prob = prob.astype(np.float16).astype(np.float32)
    o = np.zeros((64, 16), dtype=np.float32)
    for t in range(64):
        o = np.float32(o + np.float32(prob[:, t, None] * v[None, t, :]))
    return o


def fixed_tile_cases():
    """The 15 (name, Q, K, V) inputs of run_execution.py:66-68."""
    cases = []
    for seed in range(10):
        rng = np.random.default_rng(seed)
        cases.append(("seed" + str(seed),
                      *[rng.uniform(-1, 1, (64, 16)).astype(np.float16) for _ in range(3)]))
    z = np.zeros((64, 16), dtype=np.float16)
    one = np.ones_like(z)
    coord = np.linspace(-1, 1, 1024).reshape(64, 16).astype(np.float16)
    hot = z.copy()
    hot[13, 7] = 1
    cancel = np.tile(np.array([1, -1], np.float16)[:, None], (32, 16))
    cases += [("zeroQK", z, z, coord), ("constant", one, one, one),
              ("signedcoords", coord, -coord, coord), ("onehotV", coord, coord, hot),
              ("cancelV", z, z, cancel)]
    return cases
