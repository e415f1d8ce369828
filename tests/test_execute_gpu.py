"""execute(): frisk tile programs built with the builder API, run on the GPU
through the C-ABI and checked against the fp64 oracle (tolerances as in the
GEMM / attention parity tests)."""
import math

import numpy as np
import pytest
import torch

import frisk_amd as F
from oracle import attention as A
from oracle import gemm as G
from tests import programs as P
from tests.gpu_util import decode, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("dtype,out", [("bf16", "bf16"), ("fp16", "fp32")])
def test_execute_tiled_gemm(ta, tb, dtype, out):
    M, N, K = 512, 384, 640
    print(f"execute tiled gemm {dtype}->{out} ta={ta} tb={tb}", flush=True)
    s, _ = P.tiled_gemm(M, N, K, BM=128, BN=128, BK=64, dtype=dtype, out=out, trans_a=ta, trans_b=tb)
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
    a = randn((K, M) if ta else (M, K), 11).to(tdt[dtype])
    b = randn((N, K) if tb else (K, N), 12).to(tdt[dtype])
    c = torch.full((M, N), float("nan"), dtype=tdt[out], device="cuda")
    F.execute(s.module, "matmul", [a, b, c])
    torch.cuda.synchronize()
    A_ = decode(a).T if ta else decode(a)
    B_ = decode(b).T if tb else decode(b)
    err = G.row_scaled_error(decode(c), A_ @ B_)
    assert err <= (1e-2 if out != "fp32" else 1e-5), err


def test_execute_whole_gemm_accumulates():
    M, N, K = 256, 256, 128
    s, _ = P.whole_gemm(M, N, K, dtype="bf16", out="fp32", clear=False)
    a = randn((M, K), 3).to(torch.bfloat16)
    b = randn((K, N), 4).to(torch.bfloat16)
    c0 = randn((M, N), 5)
    c = c0.clone()
    F.execute(s.module, "gemm", [a, b, c])
    torch.cuda.synchronize()
    ref = decode(a) @ decode(b) + c0.double().cpu().numpy()
    assert G.row_scaled_error(decode(c), ref) <= 1e-5


@pytest.mark.parametrize("M,N,K", [(32, 2048, 16384), (512, 1024, 8192)])
def test_execute_whole_gemm_split_k(M, N, K):
    # Shapes whose frisk_gemm splits K when given a workspace (the small-M
    # kernel at M = 32 with 64 MiB of W; an under-filled tile grid at
    # M = 512): execute() passes one, and the result matches the fp64 oracle
    # on sampled rows.
    from frisk_amd import runtime as rt
    print(f"execute whole gemm split-k {M}x{N}x{K}", flush=True)
    s, _ = P.whole_gemm(M, N, K, dtype="bf16", out="bf16", trans_b=True)
    a = randn((M, K), 21).to(torch.bfloat16)
    b = randn((N, K), 22).to(torch.bfloat16)
    c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert rt.gemm_workspace_bytes(a, b, c, trans_b=True) > 0
    F.execute(s.module, "gemm", [a, b, c])
    torch.cuda.synchronize()
    rows = np.arange(0, M, max(1, M // 32))
    ref = decode(a)[rows] @ decode(b).T
    assert G.row_scaled_error(decode(c)[rows], ref) <= 1e-2


@pytest.mark.parametrize("k_transposed", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_execute_attention(k_transposed, causal):
    Bt, H, S, D = 1, 2, 256, 128
    print(f"execute attention k_transposed={k_transposed} causal={causal}", flush=True)
    s, _ = P.attention(Bt, H, S, D, k_transposed=k_transposed)
    q = randn((Bt, H, S, D), 21).to(torch.bfloat16)
    k = randn((Bt, H, S, D), 22).to(torch.bfloat16)
    v = randn((Bt, H, S, D), 23).to(torch.bfloat16)
    o = torch.full_like(q, float("nan"))
    k_arg = k.transpose(-1, -2).contiguous() if k_transposed else k
    F.execute(s.module, "attention", [q, k_arg, v, o], causal=causal)
    torch.cuda.synchronize()
    ro, _ = A.attention_fp64(decode(q), decode(k), decode(v), causal=causal, scale=1 / math.sqrt(D))
    assert G.row_scaled_error(decode(o), ro) <= 1e-2


def test_execute_checks_tensors():
    s, _ = P.whole_gemm(64, 64, 64)
    a = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="must be bf16"):
        F.execute(s.module, "gemm", [a, a, torch.zeros(64, 64, device="cuda")])
    with pytest.raises(ValueError, match="takes 3 tensors"):
        F.execute(s.module, "gemm", [a, a])
    with pytest.raises(ValueError, match="no kernel"):
        F.execute(s.module, "nope", [a, a, a])


def test_execute_config_c1_fp32_512():
    # fp32 C = A.B, M = N = K = 512, row-major A [M, K] and
    # B [K, N] ~ U[-1, 1] from a fixed seed, built as a Frisk GEMM IR with the
    # reference's helper API (FriskHelper.create_gemm, python/frisk/common/
    # utils.py:103-117) and run through execute(); checked against the fp64
    # oracle and the reference's fp32 rank-1-update oracle
    # (run_execution.py:58-63).
    s, _ = P.whole_gemm(512, 512, 512, dtype="fp32", out="fp32")
    rng = np.random.default_rng(0)
    a_np = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    b_np = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    a, b = torch.from_numpy(a_np).cuda(), torch.from_numpy(b_np).cuda()
    c = torch.full((512, 512), float("nan"), device="cuda")
    F.execute(s.module, "gemm", [a, b, c])
    torch.cuda.synchronize()
    got = c.cpu().numpy().astype(np.float64)
    assert G.row_scaled_error(got, G.gemm_fp64(a_np, b_np)) <= 1e-5
    assert G.row_scaled_error(got, G.gemm_fp32_rank1(a_np, b_np)) <= 1e-5


def test_execute_reference_fp32_tile_program():
    # The reference's GEMM tile program (tmp/ir.mlir:2-16): fp32 C = A.B at
    # 1024^3 in 128x128x32 workgroup tiles on 256 threads.  Its instruction
    # contract selects the 128x128 kernel with a 2x2 wave grid on
    # v_mfma_f32_32x32x2_f32, which execute() runs; fp32 parity against
    # the fp64 oracle.
    from frisk_amd import executor
    s, _ = P.tiled_gemm(1024, 1024, 1024, BM=128, BN=128, BK=32, dtype="fp32", out="fp32")
    p = executor.plan(s.module, "matmul")
    # 64 tiles on 256 CUs: the launch contract splits K in 4 on that tile.
    assert p.variant == (128, 2, 2, 4) and p.layouts_match, (p.contract, p.mismatch)
    assert "v_mfma_f32_32x32x2_f32" in p.contract
    rng = np.random.default_rng(1)
    a_np = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    b_np = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    a, b = torch.from_numpy(a_np).cuda(), torch.from_numpy(b_np).cuda()
    c = torch.full((1024, 1024), float("nan"), device="cuda")
    F.execute(s.module, "matmul", [a, b, c])
    torch.cuda.synchronize()
    ref = G.gemm_fp64(a_np, b_np)
    assert G.row_scaled_error(c.cpu().numpy().astype(np.float64), ref) <= 1e-5


def test_execute_falls_back_on_a_misaligned_view():
    # A 128x128-tile program whose contract selects the 128x128 kernel,
    # given an A that is a view at an odd element offset (2-byte aligned):
    # the variant's matrix-core conditions fail on these tensors, so the
    # library's own choice (the generic kernel) runs, the plan says why, and
    # the result matches the oracle.
    from frisk_amd import executor
    M = N = K = 256
    s, _ = P.tiled_gemm(M, N, K, BM=128, BN=128, BK=64, trans_b=True)
    buf = randn((M * K + 1,), 31).to(torch.bfloat16)
    a = buf[1:].view(M, K)
    b = randn((N, K), 32).to(torch.bfloat16)
    c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    p = executor.plan(s.module, "matmul")
    assert p.variant is not None and p.layouts_match
    assert executor._checked_variant(p, a, b, c) is None
    assert not p.layouts_match and "does not run on these tensors" in p.mismatch
    with pytest.raises(ValueError, match="no kernel runs the contracts"):
        F.execute(s.module, "matmul", [a, b, c], require_layout_match=True)
    F.execute(s.module, "matmul", [a, b, c])
    torch.cuda.synchronize()
    assert G.row_scaled_error(decode(c), decode(a) @ decode(b).T) <= 1e-2


@pytest.mark.parametrize("M,N,K,tb", [(4096, 4096, 4096, True), (1024, 4096, 4096, False),
                                      (128, 4096, 4096, True), (16, 4096, 14336, True)])
def test_execute_whole_gemm_runs_the_launch_contract(M, N, K, tb):
    # Whole-matrix programs take the target's launch contract (tile, wave
    # grid, K slices), request it through the C-ABI, and match the oracle.
    from frisk_amd import executor
    from frisk_amd import runtime as rt
    s, _ = P.whole_gemm(M, N, K, dtype="bf16", out="bf16", trans_b=tb)
    p = executor.plan(s.module, "gemm")
    a = randn((M, K), 41).to(torch.bfloat16)
    b = randn((N, K) if tb else (K, N), 42).to(torch.bfloat16)
    c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    if p.variant is not None:
        req = rt.gemm_plan(a, b, c, trans_b=tb, variant=p.variant)
        assert req["requested"] and req["slices"] == p.launch["slices"]
    F.execute(s.module, "gemm", [a, b, c], require_layout_match=True)
    torch.cuda.synchronize()
    rows = np.arange(0, M, max(1, M // 32))
    ref = decode(a)[rows] @ (decode(b).T if tb else decode(b))
    assert G.row_scaled_error(decode(c)[rows], ref) <= 1e-2
