"""CPU oracle of the tile ops: reduction, element-converting copy and fill.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py as the checker; the product path
(frisk_amd) never calls it.

Restated from the reference:

* `reduce` - frisk.reduce / frisk.reduce_tensor.  Kinds add(sum)/max/min
  along one axis, computed in the element type (include/Dialect/Frisk/IR/
  FriskLayoutOps.td:17-30); combine() follows the CPU contract of
  unittests/Dialect/Frisk/Layout/LegacyNormalizationNumericTest.cpp:20-30
  (NaN propagates, max(+0, -0) = +0, min(+0, -0) = -0); clear=False merges as
  combine(old, reduction) (lib/Dialect/Frisk/Transforms/
  LegacyFragmentNormalization.cpp:534-552).  Sums associate as
  canonical_fiber_tree_v1 (lib/Dialect/Frisk/Analysis/
  ReductionLayoutProof.cpp:108-140): the leaves in order, adjacent pairs
  combined level by level, an odd last node carried up unchanged.  Leaves are
  in ascending index order along the reduced axis.
* `convert` - frisk.copy of a whole tile with an element-type change
  (tmp/ir.mlir:154), i.e. arith.extf (exact) / arith.truncf (round to nearest
  even; f16/bf16 overflow to inf, e4m3fn overflow and NaN to NaN).
* `fill_bits` - a frisk.fill value as a FloatAttr of the tile's element type
  (ffi/ir.cpp:439-454), round to nearest even.

Element values are carried as float32 arrays (f32, and f16/bf16/e4m3 values,
which float32 represents exactly) or as raw bit arrays (`to_bits`,
`from_bits`).  A sum in f16/bf16 is the float32 sum rounded to the type,
which is the correctly rounded f16/bf16 sum (float32 has 24 >= 2p + 2 bits).
"""
from __future__ import annotations

import numpy as np

SUM, MAX, MIN = 0, 1, 2
KINDS = {"sum": SUM, "add": SUM, "max": MAX, "min": MIN}
DTYPES = ("f32", "f16", "bf16", "e4m3")


# ---- rounding ------------------------------------------------------------------
def round_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), nearest even; NaN -> quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_e4m3_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> OCP e4m3fn bit patterns (uint8), nearest even.  The format
    (1 sign, 4 exponent bits with bias 7, 3 mantissa bits, S.1111.111 = NaN,
    no infinity) gives: largest finite 448, quantum 2^-9 below 2^-6;
    magnitudes above 464 (448 plus half its spacing of 32) and NaN -> NaN."""
    x = np.asarray(x, dtype=np.float32)
    sign = (x.view(np.uint32) >> 24).astype(np.uint8) & 0x80
    a = np.abs(x).astype(np.float64)
    out = np.full(x.shape, 0x7F, dtype=np.uint8)
    ok = a <= 464.0  # False for NaN and inf
    sub = ok & (a < 2.0 ** -6)
    out[sub] = np.rint(a[sub] * 512.0).astype(np.uint8)  # 8 is the least normal, 0x08
    nrm = ok & ~sub
    m, e = np.frexp(a[nrm])  # a = m 2^e, m in [0.5, 1)
    q = np.rint((m * 2.0 - 1.0) * 8.0).astype(np.int64)
    ef = e.astype(np.int64) - 1 + 7
    ef = np.where(q == 8, ef + 1, ef)
    q = np.where(q == 8, 0, q)
    out[nrm] = ((ef << 3) | q).astype(np.uint8)
    return out | sign


def e4m3_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return (s * mag).astype(np.float32)


def round_to(dtype: str, x: np.ndarray) -> np.ndarray:
    """Round float32 values to `dtype`, returned as float32 values."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        with np.errstate(over="ignore", invalid="ignore"):
            return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(round_bf16_bits(x))
    if dtype == "e4m3":
        return e4m3_bits_to_f32(round_e4m3_bits(x))
    raise ValueError(dtype)


def to_bits(dtype: str, x: np.ndarray) -> np.ndarray:
    """Bit patterns of float32 values rounded to `dtype`."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.view(np.uint32).copy()
    if dtype == "f16":
        with np.errstate(over="ignore", invalid="ignore"):
            return x.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        return round_bf16_bits(x)
    if dtype == "e4m3":
        return round_e4m3_bits(x)
    raise ValueError(dtype)


def from_bits(dtype: str, b: np.ndarray) -> np.ndarray:
    if dtype == "f32":
        return np.asarray(b, dtype=np.uint32).view(np.float32)
    if dtype == "f16":
        return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(b)
    if dtype == "e4m3":
        return e4m3_bits_to_f32(b)
    raise ValueError(dtype)


def convert(src_dtype: str, dst_dtype: str, bits: np.ndarray) -> np.ndarray:
    """frisk.copy with an element-type change on raw bits -> raw bits."""
    return to_bits(dst_dtype, from_bits(src_dtype, bits))


# ---- reduction -------------------------------------------------------------------
def combine(kind: int, dtype: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """One tree node, elementwise, in `dtype` (values carried as float32)."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    if kind == SUM:
        with np.errstate(over="ignore", invalid="ignore"):
            return round_to(dtype, a + b)
    nan = np.isnan(a) | np.isnan(b)
    ua, ub = a.view(np.uint32), b.view(np.uint32)
    if kind == MAX:
        pick = np.where(a > b, a, b)
        tie = (ua & ub).view(np.float32)
    else:
        pick = np.where(a < b, a, b)
        tie = (ua | ub).view(np.float32)
    out = np.where(a == b, tie, pick)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def canonical_tree(kind: int, dtype: str, leaves: np.ndarray) -> np.ndarray:
    """Reduce the last axis of `leaves` with canonical_fiber_tree_v1: each
    level pairs nodes (0,1), (2,3), ... and carries an odd last node up
    (ReductionLayoutProof.cpp:124-136)."""
    layer = np.asarray(leaves, dtype=np.float32)
    if layer.shape[-1] == 0:
        raise ValueError("empty reduction")
    while layer.shape[-1] > 1:
        n = layer.shape[-1]
        merged = combine(kind, dtype, layer[..., 0:n - 1:2], layer[..., 1:n:2])
        if n % 2:
            merged = np.concatenate([merged, layer[..., n - 1:]], axis=-1)
        layer = merged
    return layer[..., 0]


def leaf_indices(order) -> list:
    """Reduced index held by each leaf position when tree level j combines
    along index bit order[j]: position p -> sum_j bit_j(p) << order[j]."""
    n = len(order)
    return [sum(((p >> j) & 1) << order[j] for j in range(n)) for p in range(1 << n)]


def reduce(src: np.ndarray, kind, axis: int, dtype: str, *, clear: bool = True,
           old: np.ndarray | None = None, leaf_order=None) -> np.ndarray:
    """frisk.reduce of a rank-2 float32-valued array along `axis` in `dtype`;
    returns float32 values of the result (one per remaining index).  Leaves
    are in ascending index order, or in the order `leaf_order` describes."""
    kind = KINDS[kind] if isinstance(kind, str) else kind
    src = np.asarray(src, dtype=np.float32)
    leaves = src if axis == 1 else src.T
    if leaf_order:
        leaves = leaves[:, leaf_indices(leaf_order)]
    res = canonical_tree(kind, dtype, leaves)
    if not clear:
        res = combine(kind, dtype, np.asarray(old, dtype=np.float32), res)
    return res


# ---- fill --------------------------------------------------------------------------
_FORMATS = {  # explicit mantissa bits, exponent bits, largest finite, has infinity
    "f16": (10, 5, 65504.0, True),
    "bf16": (7, 8, 3.3895313892515355e38, True),
    "f32": (23, 8, 3.4028234663852886e38, True),
    "e4m3": (3, 4, 448.0, False),
}


def fill_bits(dtype: str, value: float) -> int:
    """Bit pattern of a double rounded to nearest even in `dtype`."""
    import math
    if dtype == "f64":
        return int(np.array([value], dtype=np.float64).view(np.uint64)[0])
    if dtype in ("i8", "i32"):
        lo, hi, mask = (-128, 127, 0xFF) if dtype == "i8" else (-2 ** 31, 2 ** 31 - 1, 0xFFFFFFFF)
        if value != math.floor(value) or not lo <= value <= hi:
            raise ValueError(f"{value} is not representable as {dtype}")
        return int(value) & mask
    mant, ebits, max_finite, has_inf = _FORMATS[dtype]
    bias = (1 << (ebits - 1)) - 1
    emin = 1 - bias
    sign = (1 << (mant + ebits)) if math.copysign(1.0, value) < 0 else 0
    emask = (1 << ebits) - 1
    nan = (emask << mant) | ((1 << (mant - 1)) if has_inf else ((1 << mant) - 1))
    if math.isnan(value):
        return nan
    a = abs(value)
    if math.isinf(a):
        return sign | (emask << mant) if has_inf else sign | nan
    if a == 0.0:
        return sign
    from fractions import Fraction
    e = max(math.frexp(a)[1] - 1, emin)
    q = Fraction(2) ** (e - mant)
    n = Fraction(a) / q
    r = round(n)  # Python rounds halves to even
    mag = r * q
    if mag > Fraction(max_finite):
        return sign | (emask << mant) if has_inf else sign | nan
    if r < (1 << mant):  # subnormal (only at e == emin)
        return sign | int(r)
    if r == (2 << mant):  # rounded up into the next binade
        e, r = e + 1, 1 << mant
    return sign | ((e + bias) << mant) | (int(r) - (1 << mant))
