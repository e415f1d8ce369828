"""GEMM parity on the GPU through the C-ABI (frisk_gemm), against the fp64 /
exact-integer oracle.  Tolerances: int8 -> int32
bit-exact; f16/bf16 max|err| <= 1e-2 * ||ref row||_inf; fp8 max|err| <=
2e-2 * ||ref row||_inf and relative Frobenius <= 2e-2; f32 outputs of
16-bit inputs 1e-5 (no output rounding)."""
import itertools

import numpy as np
import pytest
import torch

from frisk_amd import runtime as rt
from oracle import gemm as G
from tests.gpu_util import Guarded, decode, fp8_per_tensor, randn, sample_rows

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 1e-2, torch.float16: 1e-2, torch.float32: 1e-5}
FP8 = torch.float8_e4m3fn


def make_operands(m, n, k, dt, ta, tb, seed):
    a_shape = (k, m) if ta else (m, k)
    b_shape = (n, k) if tb else (k, n)
    if dt == torch.int8:
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        a = torch.randint(-127, 128, a_shape, generator=g, device="cuda", dtype=torch.int8)
        b = torch.randint(-127, 128, b_shape, generator=g, device="cuda", dtype=torch.int8)
        return a, b, 1.0, 1.0
    if dt == FP8:
        a, sa = fp8_per_tensor(randn(a_shape, seed))
        b, sb = fp8_per_tensor(randn(b_shape, seed + 1))
        return a, b, sa, sb
    return randn(a_shape, seed).to(dt), randn(b_shape, seed + 1).to(dt), 1.0, 1.0


def reference(a, b, ta, tb, sa, sb, rows=None):
    A = decode(a)
    B = decode(b)
    A = A.T if ta else A
    B = B.T if tb else B
    if rows is not None:
        A = A[rows]
    if a.dtype == torch.int8:
        # |sum| <= K * 128^2 < 2^53 for K < 2^39: every partial sum of the
        # float64 product is an exact integer, in any order.
        return (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    return (A @ B) * (sa * sb)


def check(got, ref, in_dt, out_dt):
    if in_dt == torch.int8:
        assert np.array_equal(got.astype(np.int64), ref), "int8 GEMM must be bit-exact"
        return
    err = G.row_scaled_error(got, ref)
    if in_dt == FP8:
        fro = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert err <= 2e-2 and fro <= 2e-2, (err, fro)
    else:
        tol = TOL[out_dt] if out_dt != torch.float32 else TOL[torch.float32]
        assert err <= tol, err


PAIRS = [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
         (torch.float16, torch.float16), (torch.float16, torch.float32),
         (FP8, torch.bfloat16), (FP8, torch.float16), (FP8, torch.float32),
         (torch.int8, torch.int32), (torch.float32, torch.float32)]
SHAPES = [(64, 64, 64), (256, 256, 128), (300, 264, 136), (100, 72, 48), (33, 17, 40),
          (512, 256, 1024)]


@pytest.mark.parametrize("in_dt,out_dt", PAIRS, ids=lambda x: str(x).replace("torch.", ""))
@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_small_shapes_every_type_and_layout(in_dt, out_dt, ta, tb):
    for i, (m, n, k) in enumerate(SHAPES):
        print(f"case {in_dt}->{out_dt} ta={ta} tb={tb} m={m} n={n} k={k}", flush=True)
        a, b, sa, sb = make_operands(m, n, k, in_dt, ta, tb, seed=100 + i)
        c = torch.zeros(m, n, dtype=out_dt, device="cuda")
        rt.gemm(a, b, c, trans_a=ta, trans_b=tb, scale_a=sa, scale_b=sb)
        torch.cuda.synchronize()
        got = decode(c).astype(np.float64)
        ref = reference(a, b, ta, tb, sa, sb)
        ref = np.asarray(ref, dtype=np.float64) if in_dt != torch.int8 else ref
        # f32 outputs of fp32 inputs see fp32 accumulation over K.
        check(got if in_dt != torch.int8 else decode(c), ref, in_dt, out_dt)


@pytest.mark.parametrize("in_dt,out_dt,ta,tb", [(torch.bfloat16, torch.bfloat16, False, True),
                                                (torch.bfloat16, torch.bfloat16, False, False),
                                                (torch.float16, torch.float16, True, True),
                                                (FP8, torch.bfloat16, False, True),
                                                (FP8, torch.float16, True, False)],
                         ids=lambda x: str(x).replace("torch.", ""))
def test_two_rounds_of_tiles_with_edges(in_dt, out_dt, ta, tb):
    # 16 x 18 = 288 tiles of 256 x 256, more than the CUs: a second round of
    # workgroups.  The last tile row (160 rows) and column (8 columns) are
    # partial; C starts as NaN, so an output left unwritten fails too.
    m, n, k = 4000, 4360, 264
    print(f"case two rounds {in_dt}->{out_dt} ta={ta} tb={tb}", flush=True)
    a, b, sa, sb = make_operands(m, n, k, in_dt, ta, tb, seed=61)
    c = torch.full((m, n), float("nan"), dtype=out_dt, device="cuda")
    rt.gemm(a, b, c, trans_a=ta, trans_b=tb, scale_a=sa, scale_b=sb)
    torch.cuda.synchronize()
    got = decode(c).astype(np.float64)
    assert not np.isnan(got).any()
    check(got, np.asarray(reference(a, b, ta, tb, sa, sb), dtype=np.float64), in_dt, out_dt)


@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16),
                                          (torch.bfloat16, torch.float32),
                                          (torch.int8, torch.int32), (FP8, torch.float32)],
                         ids=lambda x: str(x).replace("torch.", ""))
def test_accumulate_into_c(in_dt, out_dt):
    m, n, k = 256, 264, 192
    a, b, sa, sb = make_operands(m, n, k, in_dt, False, True, seed=7)
    if out_dt == torch.int32:
        c0 = torch.randint(-1000, 1000, (m, n), dtype=torch.int32, device="cuda")
    else:
        c0 = randn((m, n), 9).to(out_dt)
    c = c0.clone()
    rt.gemm(a, b, c, trans_b=True, clear_accum=False, scale_a=sa, scale_b=sb)
    torch.cuda.synchronize()
    ref = reference(a, b, False, True, sa, sb) + decode(c0)
    check(decode(c), ref, in_dt, out_dt)


SKINNY = [(1, 64, 64), (16, 16, 8), (17, 40, 72), (48, 24, 200), (64, 4096, 512), (100, 136, 1000),
          (128, 256, 64), (128, 8200, 96),
          # single 16x16 tiles, 8 k-steps per load batch: whole batches and a K tail
          (16, 4096, 4096), (5, 40, 2056)]


@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16),
                                          (torch.bfloat16, torch.float32),
                                          (torch.float16, torch.float16)],
                         ids=lambda x: str(x).replace("torch.", ""))
@pytest.mark.parametrize("m,n,k", SKINNY)
def test_small_m_kernel(m, n, k, in_dt, out_dt):
    # M <= 128 with K-contiguous operands runs the skinny kernel: ragged N
    # (partial last tile), K tails below one 32-element step, wide N.
    print(f"case skinny m={m} n={n} k={k} {in_dt}->{out_dt}", flush=True)
    a, b, _, _ = make_operands(m, n, k, in_dt, False, True, seed=m + n + k)
    c = torch.zeros(m, n, dtype=out_dt, device="cuda")
    rt.gemm(a, b, c, trans_b=True)
    torch.cuda.synchronize()
    check(decode(c), reference(a, b, False, True, 1.0, 1.0), in_dt, out_dt)
    c0 = randn((m, n), 3).to(out_dt)
    c = c0.clone()
    rt.gemm(a, b, c, trans_b=True, clear_accum=False)
    torch.cuda.synchronize()
    check(decode(c), reference(a, b, False, True, 1.0, 1.0) + decode(c0), in_dt, out_dt)


@pytest.mark.parametrize("m,n,k", [(16, 14336, 4096), (40, 14000, 4800)])
def test_small_m_wide_tiles_unsplit(m, n, k):
    # At least 64 MiB of W in 64-column tiles that fill most CUs in one
    # round: the small-M kernel runs unsplit, with or without a workspace,
    # and asks for none (ragged M and N in the second shape).
    print(f"case skinny wide m={m} n={n} k={k}", flush=True)
    a, b, _, _ = make_operands(m, n, k, torch.bfloat16, False, True, seed=m + n + k)
    c = torch.zeros(m, n, dtype=torch.bfloat16, device="cuda")
    assert rt.gemm_workspace_bytes(a, b, c, trans_b=True) == 0
    rt.gemm(a, b, c, trans_b=True)
    torch.cuda.synchronize()
    ref = reference(a, b, False, True, 1.0, 1.0)
    check(decode(c), ref, torch.bfloat16, torch.bfloat16)
    c0 = randn((m, n), 3).to(torch.bfloat16)
    c = c0.clone()
    rt.gemm(a, b, c, trans_b=True, clear_accum=False, workspace=False)
    torch.cuda.synchronize()
    check(decode(c), ref + decode(c0), torch.bfloat16, torch.bfloat16)


BIG_RAGGED = [(4000, 2056, 1000, torch.bfloat16, torch.bfloat16),
              (4096, 4104, 776, torch.float16, torch.float32),
              (3000, 3000, 2000, FP8, torch.float32),
              (3000, 3000, 2000, FP8, torch.bfloat16),
              (4000, 2056, 1008, torch.int8, torch.int32)]


@pytest.mark.parametrize("m,n,k,in_dt,out_dt", BIG_RAGGED,
                         ids=lambda x: str(x).replace("torch.", ""))
def test_large_tiles_ragged(m, n, k, in_dt, out_dt):
    # At least 128 tiles of 256x256: the four-wave 256x256 kernel, with
    # partial edge tiles in M and N and a K tail inside the last 128-byte
    # stage; first overwriting C, then accumulating into it.
    print(f"case large m={m} n={n} k={k} {in_dt}->{out_dt}", flush=True)
    a, b, sa, sb = make_operands(m, n, k, in_dt, False, True, seed=m + k)
    r = sample_rows(m, 40, seed=k)
    rows = torch.from_numpy(r).cuda()
    ref = reference(a, b, False, True, sa, sb, rows=r)
    c = torch.empty(m, n, dtype=out_dt, device="cuda")
    rt.gemm(a, b, c, trans_b=True, scale_a=sa, scale_b=sb)
    torch.cuda.synchronize()
    check(decode(c[rows]), ref, in_dt, out_dt)
    if out_dt == torch.int32:
        c0 = torch.randint(-1000, 1000, (m, n), dtype=torch.int32, device="cuda")
    else:
        c0 = randn((m, n), 11).to(out_dt)
    c = c0.clone()
    rt.gemm(a, b, c, trans_b=True, clear_accum=False, scale_a=sa, scale_b=sb)
    torch.cuda.synchronize()
    check(decode(c[rows]), ref + decode(c0[rows]), in_dt, out_dt)


SHORT_K = [(8, torch.bfloat16, torch.bfloat16), (64, torch.bfloat16, torch.bfloat16),
           (72, torch.bfloat16, torch.float32), (136, torch.float16, torch.float16),
           (16, FP8, torch.bfloat16), (128, FP8, torch.bfloat16), (144, FP8, torch.float32),
           (272, FP8, torch.bfloat16), (16, torch.int8, torch.int32), (144, torch.int8, torch.int32)]


@pytest.mark.parametrize("k,in_dt,out_dt", SHORT_K, ids=lambda x: str(x).replace("torch.", ""))
@pytest.mark.parametrize("ta,tb", [(False, True), (True, False), (False, False)],
                         ids=["nt", "tt", "nn"])
def test_large_tiles_short_k(k, in_dt, out_dt, ta, tb):
    # 128 tiles of 256x256 over K of less than one 128-byte stage, exactly
    # one, or one or two and a tail: every iteration of the 256x256 kernel's
    # loop is a general (edge) one and its loads past the last stage read
    # zeros.
    m, n = 4096, 2048
    print(f"case short-k m={m} n={n} k={k} {in_dt}->{out_dt} ta={ta} tb={tb}", flush=True)
    a, b, sa, sb = make_operands(m, n, k, in_dt, ta, tb, seed=k + 7)
    c = torch.full((m, n), 7, dtype=out_dt, device="cuda")
    assert rt.gemm_plan(a, b, c, trans_a=ta, trans_b=tb)["kernel"] == "gemm_w4"
    rt.gemm(a, b, c, trans_a=ta, trans_b=tb, scale_a=sa, scale_b=sb)
    torch.cuda.synchronize()
    r = sample_rows(m, 48, seed=k)
    check(decode(c[torch.from_numpy(r).cuda()]), reference(a, b, ta, tb, sa, sb, rows=r),
          in_dt, out_dt)


@pytest.mark.parametrize("m,n,k", [(1024, 4096, 4096), (512, 640, 1000), (300, 1000, 72)])
def test_mid_size_tiles(m, n, k):
    # Fewer than 128 tiles of 256x256: the 128x128-tile configuration.
    print(f"case mid m={m} n={n} k={k}", flush=True)
    a, b, _, _ = make_operands(m, n, k, torch.bfloat16, False, True, seed=9)
    c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    rt.gemm(a, b, c, trans_b=True)
    torch.cuda.synchronize()
    check(decode(c), reference(a, b, False, True, 1.0, 1.0), torch.bfloat16, torch.bfloat16)


def test_sentinel_guards_and_unchanged_inputs():
    for (m, n, k), dt, odt in [((300, 264, 136), torch.bfloat16, torch.bfloat16),
                               ((300, 264, 136), torch.int8, torch.int32),
                               ((100, 136, 1000), torch.bfloat16, torch.bfloat16),
                               ((2048, 2048, 256), torch.bfloat16, torch.float32)]:
        a, b, _, _ = make_operands(m, n, k, dt, False, True, seed=11)
        a0, b0 = a.clone(), b.clone()
        gc = Guarded((m, n), odt)
        rt.gemm(a, b, gc.t, trans_b=True)
        torch.cuda.synchronize()
        assert gc.guards_intact()
        assert torch.equal(a, a0) and torch.equal(b, b0)


def run_sampled(m, n, k, in_dt, out_dt, seed, rows=48, std_a=1.0, std_b=1.0):
    """Runs the NT GEMM and checks `rows` sampled rows against the fp64
    oracle (rows=None: every output)."""
    if in_dt in (torch.bfloat16, torch.float16):
        a = randn((m, k), seed, std_a).to(in_dt)
        b = randn((n, k), seed + 1, std_b).to(in_dt)
        sa = sb = 1.0
    else:
        a, b, sa, sb = make_operands(m, n, k, in_dt, False, True, seed)
    c = torch.empty(m, n, dtype=out_dt, device="cuda")
    rt.gemm(a, b, c, trans_b=True, scale_a=sa, scale_b=sb)
    torch.cuda.synchronize()
    if rows is None:
        got, ref = decode(c), reference(a, b, False, True, sa, sb)
    else:
        r = sample_rows(m, rows, seed)
        got = decode(c[torch.from_numpy(r).cuda()])
        ref = reference(a, b, False, True, sa, sb, rows=r)
    check(got, ref, in_dt, out_dt)
    return a, b, c, sa, sb


# Small-M kernel split (M <= 64 with >= 64 MiB of W), 128x128-tile split
# (64 < M <= 128, few tiles) and 256x256-tile split (larger M), with ragged
# M, N and K tails.
SPLIT_SHAPES = [(128, 4096, 4096), (16, 2048, 16384), (100, 1000, 3000), (48, 2600, 16384),
                (1, 2048, 16384), (16, 5120, 14336), (256, 520, 8192), (300, 1000, 6144),
                (768, 2048, 4096)]


@pytest.mark.parametrize("m,n,k", SPLIT_SHAPES)
@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16),
                                          (torch.float16, torch.float32)],
                         ids=["bf16", "f16-f32"])
@pytest.mark.parametrize("accumulate", [False, True], ids=["clear", "accum"])
def test_split_k_small_m(m, n, k, in_dt, out_dt, accumulate):
    # Small-M shapes that frisk_gemm_workspace_size splits over K: the split
    # result against the fp64 oracle (C0 + A.B^T when accumulating), the
    # same call again bit for bit, and the unsplit kernel within tolerance.
    print(f"case split-k m={m} n={n} k={k} {in_dt}->{out_dt} accumulate={accumulate}", flush=True)
    a = randn((m, k), 7 + m).to(in_dt)
    b = randn((n, k), 8 + n).to(in_dt)
    assert rt.gemm_workspace_bytes(a, b, torch.empty(m, n, dtype=out_dt, device="cuda"),
                                   trans_b=True) > 0
    c0 = randn((m, n), 9).to(out_dt)
    outs = []
    for ws in (True, True, False):
        c = c0.clone()
        rt.gemm(a, b, c, trans_b=True, clear_accum=not accumulate, workspace=ws)
        torch.cuda.synchronize()
        outs.append(c)
    assert torch.equal(outs[0], outs[1])
    r = sample_rows(m, 32, m + n)
    ref = reference(a, b, False, True, 1.0, 1.0, rows=r)
    if accumulate:
        ref = ref + decode(c0[torch.from_numpy(r).cuda()])
    for c in (outs[0], outs[2]):
        check(decode(c[torch.from_numpy(r).cuda()]), ref, in_dt, out_dt)


# Split-K shapes by path: two slices of 128x128 tiles sum inside the GEMM
# launch (the arrival tree in the workspace), more slices through the
# separate slice sum; ragged M, N and K tails in both.
TREE_SHAPES = [(128, 14336, 4096), (512, 4096, 4096), (200, 6000, 3000)]
SUM_SHAPES = [(256, 4096, 4096), (128, 4096, 14336), (300, 1000, 6144)]


@pytest.mark.parametrize("m,n,k", TREE_SHAPES + SUM_SHAPES)
def test_split_k_workspace_contents_do_not_matter(m, n, k):
    # The split's result does not depend on what the workspace held before
    # the call (zeros, all-ones bytes, random bytes, or a previous call's
    # partials and arrival words): bit for bit, and within the bf16
    # tolerance of the fp64 oracle.
    print(f"case split-k workspace m={m} n={n} k={k}", flush=True)
    a = randn((m, k), 11 + m).to(torch.bfloat16)
    b = randn((n, k), 12 + n).to(torch.bfloat16)
    c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    plan = rt.gemm_plan(a, b, c, trans_b=True)
    assert plan["slices"] >= 2, plan
    need = rt.gemm_workspace_bytes(a, b, c, trans_b=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(m + n + k)
    fills = [torch.zeros(need, dtype=torch.uint8, device="cuda"),
             torch.full((need,), 0xFF, dtype=torch.uint8, device="cuda"),
             torch.randint(0, 256, (need,), generator=g, dtype=torch.uint8, device="cuda")]
    outs = []
    for ws in fills + [fills[2]]:  # the last one again: the previous call's leftovers
        rt.gemm(a, b, c, trans_b=True, workspace=ws)
        torch.cuda.synchronize()
        outs.append(c.clone())
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    r = sample_rows(m, 32, m + n)
    check(decode(outs[0][torch.from_numpy(r).cuda()]), reference(a, b, False, True, 1.0, 1.0, rows=r),
          torch.bfloat16, torch.bfloat16)


@pytest.mark.parametrize("slices", [2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("ta,tb", [(False, True), (True, False)], ids=["nt", "tn"])
def test_split_k_every_slice_count(slices, ta, tb):
    # M = 128, N = 256: 2 tiles of 128x128; K picks the slice count (8
    # stages of 128 bytes per slice at least, so K = 512 * slices bf16
    # elements gives `slices` slices).  Two slices take the in-launch tree,
    # more the separate sum; both storage orders of the operands; f32 and
    # bf16 outputs, accumulating into C.
    m, n, k = 128, 256, 512 * slices + 40
    print(f"case split-k slices={slices} ta={ta} tb={tb}", flush=True)
    a, b, _, _ = make_operands(m, n, k, torch.bfloat16, ta, tb, seed=30 + slices)
    for out_dt in (torch.float32, torch.bfloat16):
        c0 = randn((m, n), 40 + slices).to(out_dt)
        c = c0.clone()
        plan = rt.gemm_plan(a, b, c, trans_a=ta, trans_b=tb)
        assert plan["slices"] == slices, plan
        rt.gemm(a, b, c, trans_a=ta, trans_b=tb, clear_accum=False)
        torch.cuda.synchronize()
        ref = reference(a, b, ta, tb, 1.0, 1.0) + decode(c0)
        check(decode(c), ref, torch.bfloat16, out_dt)


@pytest.mark.parametrize("m,n,k", [(512, 512, 512), (1024, 1024, 1024), (300, 500, 1032)])
@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_fp32_matrix_cores_split_k(m, n, k, ta, tb):
    # fp32 on v_mfma_f32_32x32x2_f32, split over K (4 slices summed by a
    # second launch) in every storage order, accumulating into C: against
    # the fp64 oracle at 1e-5, bit-identical on a repeat, and the unsplit
    # kernel within the same tolerance.
    print(f"case f32 split m={m} n={n} k={k} ta={ta} tb={tb}", flush=True)
    if ta and m % 4:
        m += 4 - m % 4  # 16 B row pitch of an M-major A
    a, b, _, _ = make_operands(m, n, k, torch.float32, ta, tb, seed=70 + m)
    c0 = randn((m, n), 71)
    p = rt.gemm_plan(a, b, c0, trans_a=ta, trans_b=tb)
    assert p["atom"] == "v_mfma_f32_32x32x2_f32" and p["slices"] > 1, p
    outs = []
    for ws in (True, True, False):
        c = c0.clone()
        rt.gemm(a, b, c, trans_a=ta, trans_b=tb, clear_accum=False, workspace=ws)
        torch.cuda.synchronize()
        outs.append(c)
    assert torch.equal(outs[0], outs[1])
    ref = reference(a, b, ta, tb, 1.0, 1.0) + decode(c0)
    for c in (outs[0], outs[2]):
        assert G.row_scaled_error(decode(c), ref) <= 1e-5


def test_config_c1_fp32_512():
    # fp32 C = A.B, row-major A and B, U[-1, 1].
    rng = np.random.default_rng(0)
    a_np = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    b_np = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    a, b = torch.from_numpy(a_np).cuda(), torch.from_numpy(b_np).cuda()
    c = torch.empty(512, 512, device="cuda")
    rt.gemm(a, b, c)
    torch.cuda.synchronize()
    got = c.cpu().numpy().astype(np.float64)
    assert G.row_scaled_error(got, G.gemm_fp64(a_np, b_np)) <= 1e-5
    # The reference's fp32 rank-1 oracle agrees to fp32 summation error.
    assert G.row_scaled_error(got, G.gemm_fp32_rank1(a_np, b_np)) <= 1e-5


def test_config_c2_fp16_4096_nt():
    # Every output against the fp64 oracle.
    a, b, c, _, _ = run_sampled(4096, 4096, 4096, torch.float16, torch.float16, seed=2, rows=None)
    # Row checksums of every row: C.1 against A.(B^T.1) in fp64.
    ones = torch.ones(4096, 1, dtype=torch.float64, device="cuda")
    lhs = (c.double() @ ones)[:, 0]
    rhs = (a.double() @ (b.double().t() @ ones))[:, 0]
    scale = (a.double().abs() @ (b.double().abs().t() @ ones))[:, 0]
    assert float(((lhs - rhs).abs() / scale).max()) < 1e-2


@pytest.mark.parametrize("n,k", [(4096, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("m", [16, 128, 1024, 8192])
def test_config_c3_projection_sweep(m, n, k):
    # W[N, K] ~ N(0, 0.02), X[M, K] ~ N(0, 1), Y = X.W^T, bf16.
    print(f"case projection m={m} n={n} k={k}", flush=True)
    run_sampled(m, n, k, torch.bfloat16, torch.bfloat16, seed=3 + m, rows=None, std_b=0.02)


def test_config_c4_fp8():
    # e4m3 A[4096, 8192] . B[8192, 8192] (B stored [N, K]),
    # per-tensor fp32 scales, bf16 output.
    run_sampled(4096, 8192, 8192, FP8, torch.bfloat16, seed=4, rows=None)


def test_config_c4_int8_exact_with_row_checksums():
    # All 16.8M outputs exactly, then the checksums as an independent check.
    a, b, c, _, _ = run_sampled(4096, 4096, 4096, torch.int8, torch.int32, seed=5, rows=None)
    # Every row, exactly: C.1 == A.(B^T.1) in int64 (a checksum of the whole
    # product), and the checksum of checksums 1^T.C.1.
    c64 = c.cpu().numpy().astype(np.int64)
    a64 = a.cpu().numpy().astype(np.int64)
    bsum = b.cpu().numpy().astype(np.int64).sum(axis=0)
    assert np.array_equal(c64.sum(axis=1), a64 @ bsum)
    assert int(c64.sum()) == int(a64.sum(axis=0) @ b.cpu().numpy().astype(np.int64).sum(axis=0))
    assert np.array_equal(c64.sum(axis=0), (a64.sum(axis=0) @ b.cpu().numpy().astype(np.int64).T))
