"""Pins of the tile-op oracle (oracle/tileops.py) on the CPU.

* The reference's known-answer test for reductions
  (unittests/Dialect/Frisk/Layout/LegacyNormalizationNumericTest.cpp:74-118):
  every kind x clear/merge x input pair, expected values derived by hand from
  its combine() (:20-30).
* The association of sums: tree shapes derived by hand from the loop of
  ReductionLayoutProof.cpp:124-136 for small n, an independent recursive
  construction (complete power-of-two block, then the rest) for every n up to
  300, and inputs where the sequential fold of the legacy reference differs.
* Rounding: bf16 / e4m3 / f16 conversions against torch and numpy (library
  routines), and f16 / bf16 sums against exactly computed sums.
* Fill values against numpy / torch, and hand-derived ties.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import tileops as T

NAN = float("nan")


def same(a, b):
    """Equal as floats, NaN == NaN, and the sign of zero agrees."""
    a, b = np.float32(a), np.float32(b)
    if np.isnan(a) or np.isnan(b):
        return bool(np.isnan(a) and np.isnan(b))
    return bool(a == b and np.signbit(a) == np.signbit(b))


# (kind, clear, input, old) -> expected, from the reference test's combine():
# a 4x4 tile filled with `input` reduced along dim 1 (four equal leaves), then
# merged with a destination filled with `old` unless clear.
KNOWN = [
    ("add", True, 2.0, 5.0, 8.0), ("add", False, 2.0, 5.0, 13.0),
    ("add", True, -0.0, -0.0, -0.0), ("add", False, -0.0, -0.0, -0.0),
    ("add", True, 0.0, -0.0, 0.0), ("add", False, 0.0, -0.0, 0.0),
    ("add", True, NAN, 1.0, NAN), ("add", False, NAN, 1.0, NAN),
    ("add", True, 1.0, NAN, 4.0), ("add", False, 1.0, NAN, NAN),
    ("max", True, 2.0, 5.0, 2.0), ("max", False, 2.0, 5.0, 5.0),
    ("max", True, -0.0, -0.0, -0.0), ("max", False, -0.0, -0.0, -0.0),
    ("max", True, 0.0, -0.0, 0.0), ("max", False, 0.0, -0.0, 0.0),
    ("max", True, NAN, 1.0, NAN), ("max", False, NAN, 1.0, NAN),
    ("max", True, 1.0, NAN, 1.0), ("max", False, 1.0, NAN, NAN),
    ("min", True, 2.0, 5.0, 2.0), ("min", False, 2.0, 5.0, 2.0),
    ("min", True, -0.0, -0.0, -0.0), ("min", False, -0.0, -0.0, -0.0),
    ("min", True, 0.0, -0.0, 0.0), ("min", False, 0.0, -0.0, -0.0),
    ("min", True, NAN, 1.0, NAN), ("min", False, NAN, 1.0, NAN),
    ("min", True, 1.0, NAN, 1.0), ("min", False, 1.0, NAN, NAN),
]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("kind,clear,inp,old,expected", KNOWN)
def test_reference_known_answers(kind, clear, inp, old, expected, dtype):
    src = np.full((4, 4), inp, dtype=np.float32)
    res = T.reduce(src, kind, 1, dtype, clear=clear, old=np.full(4, old, dtype=np.float32))
    assert all(same(r, expected) for r in res), (res, expected)


# ---- association -----------------------------------------------------------------
def symbolic(n):
    """canonical_tree on symbols: the oracle's combine is replaced by string
    joining through the same level loop."""
    layer = [f"x{i}" for i in range(n)]
    while len(layer) > 1:
        nxt = [f"({layer[i]}+{layer[i + 1]})" for i in range(0, len(layer) - 1, 2)]
        if len(layer) % 2:
            nxt.append(layer[-1])
        layer = nxt
    return layer[0]


# Shapes obtained by executing the reference's loop (ReductionLayoutProof.cpp:
# 124-136) by hand.
HAND = {
    1: "x0", 2: "(x0+x1)", 3: "((x0+x1)+x2)", 4: "((x0+x1)+(x2+x3))",
    5: "(((x0+x1)+(x2+x3))+x4)", 6: "(((x0+x1)+(x2+x3))+(x4+x5))",
    7: "(((x0+x1)+(x2+x3))+((x4+x5)+x6))",
    11: "((((x0+x1)+(x2+x3))+((x4+x5)+(x6+x7)))+((x8+x9)+x10))",
}


@pytest.mark.parametrize("n", sorted(HAND))
def test_tree_shape_matches_the_reference_loop(n):
    assert symbolic(n) == HAND[n]


def recursive_tree(kind, dtype, x):
    """Independent construction: for n not a power of two, the first 2^k
    leaves (the largest power of two below n) form a complete subtree that is
    combined with the tree of the rest; a power of two splits in halves."""
    n = len(x)
    if n == 1:
        return np.float32(x[0])
    half = 1 << (n - 1).bit_length() - 1
    return T.combine(kind, dtype, recursive_tree(kind, dtype, x[:half]),
                     recursive_tree(kind, dtype, x[half:]))


def sensitive_values(rng, n):
    """Values whose f32 sum depends on the association: random signs and
    magnitudes spread over 2^-20 .. 2^20."""
    return (rng.standard_normal(n) * np.exp2(rng.integers(-20, 21, n))).astype(np.float32)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_tree_equals_the_recursive_construction(dtype):
    rng = np.random.default_rng(3)
    for n in range(1, 301):
        x = T.round_to(dtype, sensitive_values(rng, n))
        if dtype == "f16":
            x = np.clip(x, -6e4, 6e4)
        got = T.canonical_tree(T.SUM, dtype, x[None, :])[0]
        assert same(got, recursive_tree(T.SUM, dtype, list(x))), n


def test_tree_is_not_the_sequential_fold():
    # 1 + 2^-24 + 2^-24 + ... : the fold drops every tiny term against 1,
    # the pairwise tree adds them up first.
    x = np.array([1.0] + [2.0 ** -24] * 3, dtype=np.float32)
    fold = np.float32(0)
    for v in x:
        fold = np.float32(fold + v)
    tree = T.canonical_tree(T.SUM, "f32", x[None, :])[0]
    assert fold == np.float32(1.0)
    assert tree == np.float32(1.0) + np.float32(2.0 ** -23)  # (1 + 2^-24) rounds to 1; 2^-24+2^-24 = 2^-23


def test_axis0_is_axis1_of_the_transpose():
    rng = np.random.default_rng(5)
    x = sensitive_values(rng, 37 * 23).reshape(37, 23)
    assert np.array_equal(T.reduce(x, "sum", 0, "f32").view(np.uint32),
                          T.reduce(x.T.copy(), "sum", 1, "f32").view(np.uint32))


# ---- rounding --------------------------------------------------------------------
def sample_f32_bits(rng, n=1 << 20):
    """Random bit patterns plus every exponent with edge mantissas."""
    r = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    edges = []
    for s in (0, 1):
        for e in range(256):
            for m in (0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x10000, 0x17FFF, 0x18000, 0x7FFFFF,
                      0x80000, 0x100000, 0x0FFFFF, 0x07FFFF, 0x400000):
                edges.append((s << 31) | (e << 23) | m)
    return np.concatenate([r, np.array(edges, dtype=np.uint32)]).view(np.float32)


def test_bf16_rounding_matches_torch():
    import torch
    x = sample_f32_bits(np.random.default_rng(7))
    ours = T.round_bf16_bits(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(T.bf16_bits_to_f32(ours[nan])))


def test_e4m3_rounding_and_decode_match_torch():
    import torch
    x = sample_f32_bits(np.random.default_rng(8))
    # plus the neighbourhood of every e4m3 value and of the ties between them
    vals = T.e4m3_bits_to_f32(np.arange(256, dtype=np.uint8))
    fin = vals[np.isfinite(vals)].astype(np.float64)
    mids = np.concatenate([fin, (np.sort(fin)[1:] + np.sort(fin)[:-1]) / 2, [464.0, 480.0, 500.0]])
    near = np.concatenate([np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
                           np.nextafter(mids.astype(np.float32), np.float32(-np.inf)),
                           mids.astype(np.float32)])
    x = np.concatenate([x, near, -near])
    ours = T.round_e4m3_bits(x)
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    nan = np.isnan(T.e4m3_bits_to_f32(ref))
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7F) == 0x7F)
    dec = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    ours_dec = T.e4m3_bits_to_f32(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(dec), np.isnan(ours_dec))
    ok = ~np.isnan(dec)
    assert np.array_equal(dec[ok].view(np.uint32), ours_dec[ok].view(np.uint32))


def test_f16_rounding_is_numpy():
    x = sample_f32_bits(np.random.default_rng(9))
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    assert np.array_equal(T.to_bits("f16", x), ref.view(np.uint16))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_sums_in_dtype_are_correctly_rounded(dtype):
    """combine(sum) of two dtype values equals the exact sum rounded once to
    dtype (the exact sum is formed in float64, exact for these magnitudes)."""
    import torch
    rng = np.random.default_rng(10)
    n = 200000
    a = T.round_to(dtype, (rng.standard_normal(n) * np.exp2(rng.integers(-12, 12, n))).astype(np.float32))
    b = T.round_to(dtype, (rng.standard_normal(n) * np.exp2(rng.integers(-12, 12, n))).astype(np.float32))
    exact = a.astype(np.float64) + b.astype(np.float64)  # <= 8 + 24 + 1 bits: exact
    if dtype == "f16":
        ref = exact.astype(np.float16).astype(np.float32)
    else:
        # float64 -> bf16 through torch goes via float32, which may double
        # round; round the exact sum with Fractions instead on the ties.
        ref = torch.from_numpy(exact).to(torch.float32).to(torch.bfloat16).float().numpy()
        f32 = exact.astype(np.float32)
        inexact = f32.astype(np.float64) != exact
        for i in np.nonzero(inexact)[0]:
            ref[i] = np.float32(_round_fraction(Fraction(float(exact[i])), 7))
    got = T.combine(T.SUM, dtype, a, b)
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def _round_fraction(v: Fraction, mant: int) -> float:
    if v == 0:
        return 0.0
    s = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    q = Fraction(2) ** (e - mant)
    return s * float(round(a / q) * q)


# ---- conversion and fill ---------------------------------------------------------------
@pytest.mark.parametrize("src,dst", [(s, d) for s in T.DTYPES for d in T.DTYPES if s != d])
def test_convert_roundtrips_widening_exactly(src, dst):
    """Every value of the narrower type survives a round trip through the
    wider one; narrowing equals rounding the decoded value."""
    rng = np.random.default_rng(11)
    bits = {"f32": rng.integers(0, 1 << 32, 4096, dtype=np.uint64).astype(np.uint32),
            "f16": np.arange(1 << 16, dtype=np.uint32).astype(np.uint16),
            "bf16": np.arange(1 << 16, dtype=np.uint32).astype(np.uint16),
            "e4m3": np.arange(256, dtype=np.uint16).astype(np.uint8)}[src]
    out = T.convert(src, dst, bits)
    vals = T.from_bits(src, bits)
    assert np.array_equal(out, T.to_bits(dst, vals))
    width = {"e4m3": 0, "f16": 1, "bf16": 1, "f32": 2}
    if width[dst] > width[src] and not (src, dst) in (("f16", "bf16"), ("bf16", "f16")):
        back = T.convert(dst, src, out)
        ok = ~np.isnan(vals)
        assert np.array_equal(back[ok], bits[ok])


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
def test_fill_bits_match_library_conversions():
    import torch
    rng = np.random.default_rng(12)
    vals = list(sample_f32_bits(rng, 4000).astype(np.float64)) + [0.0, -0.0, 1e-300, -1e300,
                                                                  65519.0, 65520.0, 464.0, 465.0]
    for v in vals:
        v = float(v)
        assert T.fill_bits("f16", v) == int(np.array([v]).astype(np.float16).view(np.uint16)[0]) \
            or math.isnan(v), v
        # f32-representable doubles: torch's float path rounds once
        t = torch.tensor([v], dtype=torch.float32)
        if not math.isnan(v) and float(t[0]) == v:
            assert T.fill_bits("bf16", v) == int(t.to(torch.bfloat16).view(torch.int16)[0]) & 0xFFFF, v
            ref8 = int(t.to(torch.float8_e4m3fn).view(torch.uint8)[0])
            ours8 = T.fill_bits("e4m3", v)
            assert ours8 == ref8 or (ours8 & 0x7F == 0x7F and ref8 & 0x7F == 0x7F), v
            assert T.fill_bits("f32", v) == int(t.view(torch.int32)[0]) & 0xFFFFFFFF


def test_fill_bits_round_doubles_once():
    # 1 + 2^-8 + 2^-40 lies just above the bf16 tie 1 + 2^-8: one rounding
    # gives 1 + 2^-7 (0x3F81); rounding through f32 first would tie to 1.0.
    assert T.fill_bits("bf16", 1.0 + 2.0 ** -8 + 2.0 ** -40) == 0x3F81
    assert T.fill_bits("bf16", 1.0 + 2.0 ** -8) == 0x3F80
    assert T.fill_bits("e4m3", 464.0) == 0x7E and T.fill_bits("e4m3", -465.0) == 0xFF
    assert T.fill_bits("e4m3", 2.0 ** -10) == 0x00 and T.fill_bits("e4m3", 1.5 * 2.0 ** -10) == 0x01
    assert T.fill_bits("f16", 65520.0) == 0x7C00 and T.fill_bits("f16", 2.0 ** -25) == 0
    assert T.fill_bits("f16", 2.0 ** -25 + 2.0 ** -40) == 1
    assert T.fill_bits("i8", -128.0) == 0x80 and T.fill_bits("i32", -1.0) == 0xFFFFFFFF
    with pytest.raises(ValueError):
        T.fill_bits("i8", 1.5)


def test_leaf_order_permutes_the_leaves():
    # order [1, 0]: level 0 pairs indices (0, 2) and (1, 3)
    assert T.leaf_indices([1, 0]) == [0, 2, 1, 3]
    assert T.leaf_indices([2, 0, 1]) == [0, 4, 1, 5, 2, 6, 3, 7]
    e = 2.0 ** -24
    y = np.array([[1.0, e, 3 * e, 2 * e]], dtype=np.float32)
    # ascending: (1 + e) + (3e + 2e): 1 + e ties to 1, then 1 + 5e = 1 + 2.5 ulp -> 1 + 2 ulp
    # [1, 0]:    (1 + 3e) + (e + 2e): 1 + 1.5 ulp -> 1 + 2 ulp, then + 1.5 ulp = 3.5 ulp -> 4 ulp
    ulp = 2.0 ** -23
    assert T.reduce(y, "sum", 1, "f32")[0] == np.float32(1 + 2 * ulp)
    assert T.reduce(y, "sum", 1, "f32", leaf_order=[1, 0])[0] == np.float32(1 + 4 * ulp)
    assert T.reduce(y, "sum", 1, "f32", leaf_order=[0, 1])[0] == T.reduce(y, "sum", 1, "f32")[0]
