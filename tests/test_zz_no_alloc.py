"""frisk_gemm_noalloc (include/frisk_hip.h): the allocation-free GEMM entry
point against frisk_gemm given a caller workspace.  Both run the same
kernels with the same split-K plan and add the slices in the same order, so
the outputs must agree bit for bit.  Calls come in a row on one stream, each
smaller than the one before, so stale scratch contents from a larger call
would show up in a smaller one."""
import pytest
import torch

from frisk_amd import runtime as rt
from tests.gpu_util import randn

pytestmark = pytest.mark.gpu

# (m, n, k, trans_a, trans_b, kernel the split runs on), largest scratch
# first: 64 MiB (the whole array) on 256x256 tiles, 8 MiB on 128x128 tiles,
# 1 MiB on the small-M kernel, then a GEMM that needs no scratch at all.
CASES = [(512, 4096, 4096, False, True, "gemm_w4"),
         (128, 4096, 4096, False, False, "gemm_128"),
         (16, 4096, 14336, False, True, "gemm_skinny"),
         (1024, 1024, 1024, True, False, None)]


def operands(m, n, k, ta, tb, seed):
    a = randn((k, m) if ta else (m, k), seed).to(torch.bfloat16)
    b = randn((n, k) if tb else (k, n), seed + 1).to(torch.bfloat16)
    return a, b


@pytest.mark.parametrize("out_dt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("accumulate", [False, True], ids=["clear", "accum"])
def test_noalloc_matches_frisk_gemm_with_workspace(out_dt, accumulate):
    for i, (m, n, k, ta, tb, kernel) in enumerate(CASES):
        print(f"case noalloc m={m} n={n} k={k} ta={ta} tb={tb} out={out_dt} accumulate={accumulate}",
              flush=True)
        a, b = operands(m, n, k, ta, tb, seed=31 + i)
        c0 = randn((m, n), 7 + i).to(out_dt)
        need = rt.gemm_workspace_bytes(a, b, c0, trans_a=ta, trans_b=tb)
        assert need <= rt.NOALLOC_SCRATCH_BYTES
        p = rt.gemm_plan(a, b, c0, trans_a=ta, trans_b=tb)
        if kernel is None:
            assert need == 0 and p["slices"] == 1
        else:
            assert need > 0 and p["slices"] > 1 and p["kernel"] == kernel, p
        want = c0.clone()
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
        rt.gemm(a, b, want, trans_a=ta, trans_b=tb, clear_accum=not accumulate, workspace=ws)
        got = c0.clone()
        rt.gemm_noalloc(a, b, got, trans_a=ta, trans_b=tb, clear_accum=not accumulate)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"case {i}: noalloc differs from frisk_gemm"


def test_noalloc_repeated_on_one_stream():
    # Two calls in a row on the caller's stream, the second smaller: each
    # result equals the workspace path's.
    s = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(s):
        for m, n, k in ((512, 4096, 4096), (256, 2048, 4096)):
            a, b = operands(m, n, k, False, True, seed=m)
            c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
            rt.gemm_noalloc(a, b, c, trans_b=True, stream=s)
            outs.append((a, b, c))
    s.synchronize()
    for a, b, c in outs:
        want = torch.empty_like(c)
        rt.gemm(a, b, want, trans_b=True, workspace=True)
        torch.cuda.synchronize()
        assert torch.equal(c, want)
