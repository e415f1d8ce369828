"""Pins the GEMM oracle (oracle/gemm.py, oracle/oracle.c) independently of
the formulas it restates: brute force on tiny shapes, closed forms, the
numpy library product, exact integer arithmetic and the OCP FP8 spec."""
import itertools

import numpy as np
import pytest

from oracle import gemm as G


def brute(a, b, ta, tb):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    m = a.shape[1] if ta else a.shape[0]
    k = a.shape[0] if ta else a.shape[1]
    n = b.shape[0] if tb else b.shape[1]
    c = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            s = 0.0
            for t in range(k):
                s += (a[t, i] if ta else a[i, t]) * (b[j, t] if tb else b[t, j])
            c[i, j] = s
    return c


@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_fp64_matches_brute_force_every_layout(ta, tb):
    rng = np.random.default_rng(1)
    m, n, k = 5, 7, 3
    a = rng.standard_normal((k, m) if ta else (m, k))
    b = rng.standard_normal((n, k) if tb else (k, n))
    np.testing.assert_allclose(G.gemm_fp64(a, b, trans_a=ta, trans_b=tb), brute(a, b, ta, tb),
                               rtol=1e-13, atol=1e-13)


def test_fp64_closed_forms():
    rng = np.random.default_rng(2)
    b = rng.standard_normal((16, 9))
    np.testing.assert_array_equal(G.gemm_fp64(np.eye(16), b), b)  # I.B = B
    ones = np.ones((4, 32))
    np.testing.assert_array_equal(G.gemm_fp64(ones, np.ones((32, 6))), np.full((4, 6), 32.0))
    u, v = rng.standard_normal((8, 1)), rng.standard_normal((1, 5))
    np.testing.assert_allclose(G.gemm_fp64(u, v), u * v, rtol=0, atol=0)  # rank-1 outer product
    # transpose identity: (A.B)^T = B^T.A^T
    a = rng.standard_normal((6, 4))
    np.testing.assert_allclose(G.gemm_fp64(a, b[:4], trans_a=False).T,
                               G.gemm_fp64(b[:4], a, trans_a=True, trans_b=True), rtol=1e-14)


def test_fp64_accumulate_reads_c():
    rng = np.random.default_rng(3)
    a, b, c = rng.standard_normal((3, 4)), rng.standard_normal((4, 5)), rng.standard_normal((3, 5))
    np.testing.assert_allclose(G.gemm_fp64(a, b, c=c, clear_accum=False), a @ b + c, rtol=1e-14)


def test_fp64_matches_numpy_library_product():
    rng = np.random.default_rng(4)
    a, b = rng.standard_normal((64, 96)), rng.standard_normal((80, 96))
    np.testing.assert_allclose(G.gemm_fp64(a, b, trans_b=True), np.matmul(a, b.T), rtol=1e-12,
                               atol=1e-12)


def test_fp32_rank1_order_and_bound():
    rng = np.random.default_rng(5)
    # Small integers: every fp32 product and partial sum is exact.
    a = rng.integers(-8, 9, (7, 13)).astype(np.float32)
    b = rng.integers(-8, 9, (13, 5)).astype(np.float32)
    np.testing.assert_array_equal(G.gemm_fp32_rank1(a, b), brute(a, b, False, False))
    # General inputs: within the sequential-summation bound K * eps32 * sum|a||b|.
    a = rng.uniform(-1, 1, (16, 64)).astype(np.float32)
    b = rng.uniform(-1, 1, (64, 16)).astype(np.float32)
    got = G.gemm_fp32_rank1(a, b).astype(np.float64)
    bound = 64 * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b))
    assert np.all(np.abs(got - brute(a, b, False, False)) <= bound)
    # A sum order that differs from the rank-1 order is detectable: the
    # reversed-k product differs in some element.
    rev = G.gemm_fp32_rank1(a[:, ::-1], b[::-1, :])
    assert not np.array_equal(rev, G.gemm_fp32_rank1(a, b))


def test_int_gemm_exact():
    rng = np.random.default_rng(6)
    a = rng.integers(-127, 128, (6, 9))
    b = rng.integers(-127, 128, (5, 9))
    c = G.gemm_int(a.astype(np.int8), b.astype(np.int8), trans_b=True)
    expect = [[sum(int(a[i, t]) * int(b[j, t]) for t in range(9)) for j in range(5)] for i in range(6)]
    assert c.tolist() == expect
    # Extreme values: 4096 * 127 * 127 is exact and inside int32.
    big = G.gemm_int(np.full((2, 4096), -127, np.int8), np.full((4096, 2), -127, np.int8))
    assert int(big[0, 0]) == 4096 * 127 * 127 < 2 ** 31


def test_e4m3fn_table_against_spec_and_library():
    import torch
    t = G.e4m3fn_decode_table()
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0  # largest finite
    assert t[0x01] == 2.0 ** -9 and t[0x08] == 2.0 ** -6  # min subnormal / min normal
    assert t[0x38] == 1.0 and t[0x00] == 0.0 and np.signbit(t[0x80])
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF]) and np.isfinite(np.delete(t, [0x7F, 0xFF])).all()
    lib = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    np.testing.assert_array_equal(t, lib)


def test_bf16_decode():
    import torch
    x = torch.randn(1000).to(torch.bfloat16)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(G.bf16_decode(bits), x.double().numpy())


def test_row_scaled_error():
    ref = np.array([[1.0, -4.0], [0.0, 0.0]])
    got = np.array([[1.04, -4.0], [0.0, 0.5]])
    # row 0: 0.04 / 4; row 1 has norm 0 and is measured absolutely
    assert G.row_scaled_error(got, ref) == pytest.approx(0.5)


@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_c_oracle_matches_numpy_oracle(native_oracle, ta, tb):
    rng = np.random.default_rng(7)
    m, n, k = 33, 17, 45
    a = rng.standard_normal((k, m) if ta else (m, k))
    b = rng.standard_normal((n, k) if tb else (k, n))
    np.testing.assert_allclose(native_oracle.gemm_f64(a, b, trans_a=ta, trans_b=tb),
                               G.gemm_fp64(a, b, trans_a=ta, trans_b=tb), rtol=1e-13, atol=1e-12)
