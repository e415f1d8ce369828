"""Pins the attention oracle (oracle/attention.py, oracle/oracle.c):
the reference's own known-answer tests (ordered FP32 tree, analytic
fixtures, neutral extension, cancelV), brute force on tiny inputs and the
library softmax."""
import struct

import numpy as np
import pytest

from oracle import attention as A


def rn32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def balanced(values):
    if len(values) == 1:
        return values[0]
    mid = len(values) // 2
    return rn32(balanced(values[:mid]) + balanced(values[mid:]))


@pytest.mark.parametrize("n", (64, 65, 128, 129, 191, 192, 193, 512, 513, 1025))
def test_ordered_sum_matches_recursive_fp32_tree(n):
    # Known-answer test of test_tail_attention_reference.py:77-88.
    # Same draw sequence as the reference test: one generator, lengths in order.
    lengths = [64, 65, 128, 129, 191, 192, 193, 512, 513, 1025]
    rng = np.random.default_rng(4)
    for size in lengths[: lengths.index(n) + 1]:
        data = np.exp2(rng.integers(-24, 1, size).astype(np.float32))
    lanes = []
    for lane in range(4):
        vals = [float(x) for i, x in enumerate(data) if i // 2 % 4 == lane]
        width = 1 << (len(vals) - 1).bit_length()
        lanes.append(balanced(vals + [0.0] * (width - len(vals))))
    expect = rn32(rn32(lanes[0] + lanes[1]) + rn32(lanes[2] + lanes[3]))
    assert A.ordered_sum(data)[0] == expect


@pytest.mark.parametrize("n", (64, 65, 128, 129, 191, 192, 193, 512, 513, 1025))
@pytest.mark.parametrize("name", A.EXACT)
def test_analytic_fixtures_bitwise(n, name):
    # test_tail_attention_reference.py:90-100: the strict oracle reproduces
    # the closed forms bit for bit.
    q, k, v = A.fixture_inputs((2, 2, n, 64), name)
    strict = A.tile_oracle(q, k, v, "strict")
    exact = A.analytical(v, name, fp64=False)
    assert np.array_equal(strict.view(np.uint32), exact.view(np.uint32))
    fp64 = A.tile_oracle(q, k, v, "fp64")
    np.testing.assert_allclose(fp64, A.analytical(v, name, fp64=True), rtol=A.ERROR["fp64_rtol"],
                               atol=A.ERROR["fp64_atol"])
    if name == "last-key-dominant":
        assert not np.array_equal(strict[..., 0, :], strict[..., -1, :])


def test_neutral_extension_is_bitwise_invariant():
    # test_tail_attention_reference.py:102-119 / tail_attention_reference.py:
    # 168-187: keys with logit -8192 and V = -32768 leave earlier outputs
    # unchanged, and tail queries copy query 0.
    rng = np.random.default_rng(14261107)
    for base, tail in ((128, 129), (192, 193), (512, 513)):
        shape = (1, 2, tail, 64)
        q, k, v = (np.zeros(shape, dtype=np.float16) for _ in range(3))
        t = rng.integers(-4, 5, (1, 2, 4, 64)).astype(np.float32) / 32
        q[..., :base, :] = t[..., np.arange(base) % 4, :]
        k[..., :base, :] = rng.integers(-4, 5, (1, 2, base, 64)).astype(np.float32) / 32
        v[..., :base, :] = rng.integers(1, 8, (1, 2, base, 64)).astype(np.float32) / 16
        q[..., :base, 0] = 1
        k[..., :base, 0] = 0
        q[..., base:, :] = q[..., :1, :]
        k[..., base:, 0] = -8192
        v[..., base:, :] = -32768
        full = A.tile_oracle(q, k, v, "strict")
        short = A.tile_oracle(q[..., :base, :], k[..., :base, :], v[..., :base, :], "strict")
        assert np.array_equal(full[..., :base, :].view(np.uint32), short.view(np.uint32))
        assert np.array_equal(full[..., base:, :], np.broadcast_to(full[..., :1, :],
                                                                    full[..., base:, :].shape))


def test_fixed_tile_cases_and_cancel():
    cases = A.fixed_tile_cases()
    assert [c[0] for c in cases][-5:] == ["zeroQK", "constant", "signedcoords", "onehotV",
                                         "cancelV"] and len(cases) == 15
    name, q, k, v = cases[-1]
    # test_numerical_cases.py:5-9: V cancels along keys, P is uniform.
    assert np.all(v.astype(np.float32).sum(axis=0) == 0)
    assert np.array_equal(A.fixed_tile_reference(q, k, v), np.zeros((64, 16), np.float32))
    # Every case agrees with the fp64 oracle at the reference's own bound
    # (run_execution.py:85: |got - ref| <= .002 + .002 |ref|), with the 0.25
    # score scale of the fixture.
    for name, q, k, v in cases:
        ref = A.fixed_tile_reference(q, k, v)
        o, _ = A.attention_fp64(q[None, None], k[None, None], v[None, None], scale=0.25)
        assert np.all(np.abs(o[0, 0] - ref) <= 0.002 + 0.002 * np.abs(ref) + 2e-3), name


def brute_attention(q, k, v, causal, scale):
    sq, d = q.shape
    sk = k.shape[0]
    o = np.zeros((sq, d))
    lse = np.zeros(sq)
    for i in range(sq):
        s = []
        for j in range(sk):
            if causal and j > i + sk - sq:
                continue
            s.append((j, scale * sum(q[i, x] * k[j, x] for x in range(d))))
        mx = max(val for _, val in s)
        den = sum(np.exp(val - mx) for _, val in s)
        for j, val in s:
            o[i] += np.exp(val - mx) / den * v[j]
        lse[i] = np.log(den) + mx
    return o, lse


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(5, 5), (4, 7), (6, 3)])
def test_fp64_attention_brute_force(causal, sq, sk):
    rng = np.random.default_rng(8)
    d = 4
    q, k, v = rng.standard_normal((sq, d)), rng.standard_normal((sk, d)), rng.standard_normal((sk, d))
    if causal and sq > sk:
        sq_eff = sk  # rows without a visible key are checked separately
        q = q[-sq_eff:]
        sq = sq_eff
    o, lse = A.attention_fp64(q[None, None], k[None, None], v[None, None], causal=causal, scale=0.7)
    bo, bl = brute_attention(q, k, v, causal, 0.7)
    np.testing.assert_allclose(o[0, 0], bo, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse[0, 0], bl, rtol=1e-12, atol=1e-12)


def test_fp64_attention_closed_forms_and_library():
    import torch
    rng = np.random.default_rng(9)
    q = np.zeros((1, 1, 8, 16))
    k = rng.standard_normal((1, 1, 8, 16))
    v = rng.standard_normal((1, 1, 8, 16))
    o, lse = A.attention_fp64(q, k, v)
    np.testing.assert_allclose(o[0, 0], np.broadcast_to(v[0, 0].mean(axis=0), (8, 16)), rtol=1e-13)
    np.testing.assert_allclose(lse, np.log(8.0), rtol=1e-14)  # Q = 0: ln(#keys)
    o, lse = A.attention_fp64(q, k, v, causal=True)
    np.testing.assert_allclose(o[0, 0, 0], v[0, 0, 0], rtol=0, atol=1e-15)  # causal row 0 = V[0]
    np.testing.assert_allclose(lse[0, 0], np.log(np.arange(1, 9)), rtol=1e-14)
    # Rows with no visible key (causal, seq_q > seq_k): O = 0, LSE = -inf.
    o, lse = A.attention_fp64(rng.standard_normal((1, 1, 5, 4)), k[..., :3, :4], v[..., :3, :4],
                              causal=True)
    assert np.all(o[0, 0, :2] == 0) and np.all(np.isneginf(lse[0, 0, :2]))
    # Library softmax.
    q = rng.standard_normal((2, 3, 33, 16))
    k = rng.standard_normal((2, 3, 40, 16))
    v = rng.standard_normal((2, 3, 40, 16))
    o, lse = A.attention_fp64(q, k, v, scale=0.3)
    s = torch.from_numpy(q) @ torch.from_numpy(k).transpose(-1, -2) * 0.3
    np.testing.assert_allclose(o, (torch.softmax(s, -1) @ torch.from_numpy(v)).numpy(), rtol=1e-12,
                               atol=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(s, -1).numpy(), rtol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_c_oracle_matches_numpy_oracle(native_oracle, causal):
    rng = np.random.default_rng(10)
    q = rng.standard_normal((1, 1, 70, 32))
    k = rng.standard_normal((1, 1, 90, 32))
    v = rng.standard_normal((1, 1, 90, 32))
    o, lse = A.attention_fp64(q, k, v, causal=causal)
    co, cl = native_oracle.attn_f64(q[0, 0], k[0, 0], v[0, 0], causal=causal)
    np.testing.assert_allclose(co, o[0, 0], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(cl, lse[0, 0], rtol=1e-13)


@pytest.mark.parametrize("causal", [False, True])
def test_c_row_subset_oracle_matches_numpy_oracle(native_oracle, causal):
    # Selected rows, each with its own causal mask (seq_k > seq_q, so the
    # mask is offset by seq_k - seq_q), in any order, against the numpy
    # oracle's rows; row 0 and the last row included.
    rng = np.random.default_rng(12)
    q = rng.standard_normal((1, 1, 70, 32))
    k = rng.standard_normal((1, 1, 90, 32))
    v = rng.standard_normal((1, 1, 90, 32))
    o, lse = A.attention_fp64(q, k, v, causal=causal)
    rows = np.array([69, 0, 17, 5, 40])
    co, cl = native_oracle.attn_rows_f64(q[0, 0], k[0, 0], v[0, 0], rows, causal=causal)
    np.testing.assert_allclose(co, o[0, 0][rows], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(cl, lse[0, 0][rows], rtol=1e-13)
