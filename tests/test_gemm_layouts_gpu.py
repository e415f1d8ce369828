"""GEMM parity on the matrix cores for every storage order of A and B.

frisk.gemm takes A as [M, K] or, with transA, [K, M], and B as [K, N] or,
with transB, [N, K] (ffi/ir.cpp:335-337).  The builder's default
transA = transB = False and the reference's own GEMM tile program
(tmp/ir.mlir:2-16, B tile memref<32x128> = [K, N]) keep B K-by-N.  Every case
here first asserts (frisk_gemm_plan) that the launch runs an MFMA kernel, not
the generic fallback, then checks the result against the fp64 / exact
integer oracle with the north-star tolerances: int8 bit-exact, f16/bf16
max|err| <= 1e-2 ||ref row||_inf, fp8 2e-2 (plus relative Frobenius)."""
import itertools

import numpy as np
import pytest
import torch

from frisk_amd import runtime as rt
from tests.gpu_util import Guarded, decode, randn, sample_rows
from tests.test_gemm_gpu import FP8, check, make_operands, reference

pytestmark = pytest.mark.gpu

LAYOUTS = list(itertools.product([False, True], repeat=2))
LAYOUT_IDS = [f"ta{int(a)}tb{int(b)}" for a, b in LAYOUTS]
MFMA_PAIRS = [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
              (torch.float16, torch.float16), (torch.float16, torch.float32),
              (FP8, torch.bfloat16), (FP8, torch.float16), (FP8, torch.float32),
              (torch.int8, torch.int32)]
PAIR_IDS = [f"{str(i).replace('torch.', '')}-{str(o).replace('torch.', '')}" for i, o in MFMA_PAIRS]


def run(a, b, c, ta, tb, sa=1.0, sb=1.0, kernel=None, **kw):
    p = rt.gemm_plan(a, b, c, trans_a=ta, trans_b=tb, workspace=kw.get("workspace", True))
    assert p["kernel"] != "gemm_generic", p
    if kernel is not None:
        assert p["kernel"] == kernel, p
    rt.gemm(a, b, c, trans_a=ta, trans_b=tb, scale_a=sa, scale_b=sb, **kw)
    torch.cuda.synchronize()
    return p


# (m, n, k, kernel, stage bytes): 256x256 tiles (at least 128 of them) with
# ragged edges in M and N and a K tail inside the last stage; 128x128 tiles
# likewise, on a grid of at most one workgroup per CU (128-byte stages) and
# on a larger one (299 tiles: 64-byte stages, two workgroups per CU).
# Every extent keeps 16 B row pitches for 8-bit M/N-major storage.
SHAPES = [(2064, 4000, 1008, "gemm_w4", 128), (304, 528, 784, "gemm_128", 128),
          (1552, 2832, 528, "gemm_128", 64)]


@pytest.mark.parametrize("in_dt,out_dt", MFMA_PAIRS, ids=PAIR_IDS)
@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
@pytest.mark.parametrize("m,n,k,kernel,stage", SHAPES, ids=["w4", "t128", "t128s64"])
def test_every_layout_and_type_on_mfma(m, n, k, kernel, stage, in_dt, out_dt, ta, tb):
    print(f"case layout ta={ta} tb={tb} {in_dt}->{out_dt} m={m} n={n} k={k}", flush=True)
    a, b, sa, sb = make_operands(m, n, k, in_dt, ta, tb, seed=m + n + 3 * ta + 5 * tb)
    c = torch.empty(m, n, dtype=out_dt, device="cuda")
    p = run(a, b, c, ta, tb, sa, sb, kernel=kernel, workspace=False)
    assert p["stage_bytes"] == stage, p
    assert p["a_major"] == ("m" if ta else "k") and p["b_major"] == ("k" if tb else "n")
    r = sample_rows(m, 48, seed=k) if kernel == "gemm_w4" else None
    ref = reference(a, b, ta, tb, sa, sb, rows=r)
    got = decode(c if r is None else c[torch.from_numpy(r).cuda()])
    check(got, ref, in_dt, out_dt)


@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16),
                                          (torch.int8, torch.int32), (FP8, torch.float32)],
                         ids=["bf16", "i8", "fp8-f32"])
def test_accumulate_every_layout(in_dt, out_dt, ta, tb):
    m, n, k = 272, 400, 560
    print(f"case accumulate ta={ta} tb={tb} {in_dt}", flush=True)
    a, b, sa, sb = make_operands(m, n, k, in_dt, ta, tb, seed=17)
    if out_dt == torch.int32:
        c0 = torch.randint(-1000, 1000, (m, n), dtype=torch.int32, device="cuda")
    else:
        c0 = randn((m, n), 9).to(out_dt)
    c = c0.clone()
    run(a, b, c, ta, tb, sa, sb, clear_accum=False)
    check(decode(c), reference(a, b, ta, tb, sa, sb) + decode(c0), in_dt, out_dt)


@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
def test_k_tail_of_mn_major_operands(ta, tb):
    # With both operands M/N-major the K tail is handled per k-row, so any
    # K runs on the matrix cores; with a K-major operand K * 2 % 16 == 0.
    m, n = 2064, 4000
    for k in ((1, 7, 65, 1001) if (ta and not tb) else (8, 72, 1000)):
        print(f"case k-tail ta={ta} tb={tb} k={k}", flush=True)
        a, b, _, _ = make_operands(m, n, k, torch.bfloat16, ta, tb, seed=k)
        c = torch.empty(m, n, dtype=torch.float32, device="cuda")
        run(a, b, c, ta, tb, workspace=False)
        r = sample_rows(m, 32, seed=k)
        check(decode(c[torch.from_numpy(r).cuda()]), reference(a, b, ta, tb, 1, 1, rows=r),
              torch.bfloat16, torch.float32)


@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
def test_strided_views_and_ragged_n(ta, tb):
    # Operands viewed out of wider buffers (row pitch > extent), and N not a
    # multiple of 8 (the epilogue's element-wise tail) with C's pitch padded.
    m, n, k = 1000, 2090, 1000
    pad = 136
    print(f"case strided ta={ta} tb={tb}", flush=True)
    ab = randn((k, m + pad) if ta else (m, k + pad), 5).to(torch.bfloat16)
    bb = randn((n, k + pad) if tb else (k, n + 6 + pad), 6).to(torch.bfloat16)
    a = ab[:, :m] if ta else ab[:, :k]
    b = bb[:, :k] if tb else bb[:, :n]
    cb = torch.full((m, n + 14), 7.0, dtype=torch.bfloat16, device="cuda")
    c = cb[:, :n]
    run(a, b, c, ta, tb, workspace=False)
    check(decode(c), reference(a, b, ta, tb, 1, 1), torch.bfloat16, torch.bfloat16)
    assert torch.all(cb[:, n:] == 7.0), "wrote past the ragged last column"


SPLIT = [(128, 4096, 4096, "gemm_128"), (384, 4096, 8192, "gemm_w4"), (100, 1000, 3000, "gemm_128")]


@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
@pytest.mark.parametrize("m,n,k,kernel", SPLIT, ids=["128s", "w4s", "ragged"])
def test_split_k_every_layout(m, n, k, kernel, ta, tb):
    # Split-K slices on either tile size: bit-identical on a repeat, and
    # within tolerance of the oracle (and of the unsplit kernel).
    if (ta or tb) and m == 100:
        m = 104  # 16 B row pitch of an M-major A
    print(f"case split ta={ta} tb={tb} m={m} n={n} k={k}", flush=True)
    a, b, _, _ = make_operands(m, n, k, torch.bfloat16, ta, tb, seed=m + k)
    c0 = randn((m, n), 9).to(torch.bfloat16)
    outs = []
    for ws in (True, True, False):
        c = c0.clone()
        p = run(a, b, c, ta, tb, clear_accum=False, workspace=ws)
        if ws:
            assert p["slices"] > 1 and p["kernel"] == kernel, p
        outs.append(c)
    assert torch.equal(outs[0], outs[1])
    r = sample_rows(m, 32, m + n)
    ref = reference(a, b, ta, tb, 1.0, 1.0, rows=r) + decode(c0[torch.from_numpy(r).cuda()])
    for c in (outs[0], outs[2]):
        check(decode(c[torch.from_numpy(r).cuda()]), ref, torch.bfloat16, torch.bfloat16)


@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
def test_bf16_4096_every_layout_full_matrix(ta, tb):
    # The headline shape in each storage order, every output against fp64.
    print(f"case bf16 4096^3 ta={ta} tb={tb}", flush=True)
    a, b, _, _ = make_operands(4096, 4096, 4096, torch.bfloat16, ta, tb, seed=41)
    c = torch.empty(4096, 4096, dtype=torch.bfloat16, device="cuda")
    run(a, b, c, ta, tb, kernel="gemm_w4")
    check(decode(c), reference(a, b, ta, tb, 1.0, 1.0), torch.bfloat16, torch.bfloat16)


@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
def test_int8_4096_every_layout_exact(ta, tb):
    # configs[3] int8 4096^3, all 16.8M outputs exactly: an fp64 BLAS
    # product of int8 values is exact (|sum| <= 4096 * 127^2 < 2^53).
    print(f"case int8 4096^3 ta={ta} tb={tb}", flush=True)
    a, b, _, _ = make_operands(4096, 4096, 4096, torch.int8, ta, tb, seed=43)
    c = torch.empty(4096, 4096, dtype=torch.int32, device="cuda")
    run(a, b, c, ta, tb, kernel="gemm_w4")
    A = a.cpu().numpy().astype(np.float64)
    B = b.cpu().numpy().astype(np.float64)
    ref = (A.T if ta else A) @ (B.T if tb else B)
    assert np.array_equal(c.cpu().numpy().astype(np.float64), ref)


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (True, True)],
                         ids=["ta0tb0", "ta1tb0", "ta1tb1"])
def test_fp8_config_shape_other_layouts(ta, tb):
    # configs[3] fp8 A[4096, 8192] . B[8192, 8192] with B [K, N] / A [K, M].
    m, n, k = 4096, 8192, 8192
    print(f"case fp8 config ta={ta} tb={tb}", flush=True)
    a, b, sa, sb = make_operands(m, n, k, FP8, ta, tb, seed=4)
    c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    run(a, b, c, ta, tb, sa, sb, kernel="gemm_w4")
    r = sample_rows(m, 32, seed=4)
    check(decode(c[torch.from_numpy(r).cuda()]), reference(a, b, ta, tb, sa, sb, rows=r),
          FP8, torch.bfloat16)


@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
def test_sentinel_guards_every_layout(ta, tb):
    for (m, n, k), dt, odt in [((304, 264, 144), torch.bfloat16, torch.bfloat16),
                               ((304, 272, 144), torch.int8, torch.int32),
                               ((2064, 2048, 256), torch.bfloat16, torch.float32)]:
        a, b, sa, sb = make_operands(m, n, k, dt, ta, tb, seed=11)
        a0, b0 = a.clone(), b.clone()
        gc = Guarded((m, n), odt)
        run(a, b, gc.t, ta, tb, sa, sb)
        assert gc.guards_intact()
        assert torch.equal(a, a0) and torch.equal(b, b0)


VARIANTS = [(256, 2, 2), (128, 2, 2), (128, 4, 1), (128, 1, 4), (128, 2, 1), (128, 1, 2)]


@pytest.mark.parametrize("variant", VARIANTS, ids=[f"t{t}w{a}x{b}" for t, a, b in VARIANTS])
@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16), (FP8, torch.float32),
                                          (torch.int8, torch.int32)], ids=["bf16", "fp8", "i8"])
@pytest.mark.parametrize("ta,tb", LAYOUTS, ids=LAYOUT_IDS)
def test_requested_kernel_variants(variant, in_dt, out_dt, ta, tb):
    # frisk_gemm_desc.tile / wave_m / wave_n: the tile and wave grid a tile
    # program's instruction contract names.  The plan reports exactly that
    # variant, and the result matches the oracle like the library's own choice.
    m, n, k = 304, 528, 784
    tile, wm, wn = variant
    print(f"case variant {variant} ta={ta} tb={tb} {in_dt}", flush=True)
    a, b, sa, sb = make_operands(m, n, k, in_dt, ta, tb, seed=tile + 7 * wm + 3 * wn)
    c = torch.empty(m, n, dtype=out_dt, device="cuda")
    p = rt.gemm_plan(a, b, c, trans_a=ta, trans_b=tb, variant=variant)
    assert p["requested"] and p["tile_m"] == tile and p["waves"] == [wm, wn], p
    assert p["kernel"] == ("gemm_w4" if tile == 256 else "gemm_128") and p["slices"] == 1
    assert f"wave_grid = [{wm}, {wn}]" in p["mma_contract"]
    rt.gemm(a, b, c, trans_a=ta, trans_b=tb, scale_a=sa, scale_b=sb, variant=variant)
    torch.cuda.synchronize()
    if in_dt == torch.int8:
        A = a.cpu().numpy().astype(np.float64)
        B = b.cpu().numpy().astype(np.float64)
        assert np.array_equal(c.cpu().numpy().astype(np.float64), (A.T if ta else A) @ (B.T if tb else B))
    else:
        check(decode(c), reference(a, b, ta, tb, sa, sb), in_dt, out_dt)


def test_variants_agree_bitwise_on_one_grid():
    # Every 128x128 wave grid sums each output over the same k order, so the
    # grids give identical bits (only the placement of work differs); so does
    # the library's own launch of this grid (20 tiles: 128-byte stages, where
    # the requested variants run 64-byte stages).
    m, n, k = 512, 640, 1024
    a, b, _, _ = make_operands(m, n, k, torch.bfloat16, False, True, seed=5)
    outs = []
    for v in VARIANTS[1:] + [None]:
        c = torch.empty(m, n, dtype=torch.float32, device="cuda")
        if v is None:
            p = rt.gemm_plan(a, b, c, trans_b=True, workspace=False)
            assert p["kernel"] == "gemm_128" and p["stage_bytes"] == 128, p
        rt.gemm(a, b, c, trans_b=True, variant=v, workspace=False)
        outs.append(c)
    torch.cuda.synchronize()
    for c in outs[1:]:
        assert torch.equal(c, outs[0])

