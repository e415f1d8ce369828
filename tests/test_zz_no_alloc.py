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

# (m, n, k, trans_a, trans_b, kernel the split runs on, slices), largest
# scratch first: 64 MiB (the whole array) on 256x256 tiles through the
# separate slice sum, 16 MiB on 128x128 tiles through the slice sum,
# 14 MiB on 128x128 tiles summed inside the launch (two slices, with
# arrival words), 1 MiB on the small-M kernel, then a GEMM that needs no
# scratch at all.
CASES = [(1024, 4096, 14336, False, True, "gemm_w4", 4),
         (128, 4096, 4096, False, False, "gemm_128", 8),
         (128, 14336, 4096, True, True, "gemm_128", 2),
         (16, 2048, 16384, False, True, "gemm_skinny", 8),
         (1024, 1024, 1024, True, False, None, 1)]


def operands(m, n, k, ta, tb, seed):
    a = randn((k, m) if ta else (m, k), seed).to(torch.bfloat16)
    b = randn((n, k) if tb else (k, n), seed + 1).to(torch.bfloat16)
    return a, b


@pytest.mark.parametrize("out_dt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("accumulate", [False, True], ids=["clear", "accum"])
def test_noalloc_matches_frisk_gemm_with_workspace(out_dt, accumulate):
    for i, (m, n, k, ta, tb, kernel, slices) in enumerate(CASES):
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
            assert need > 0 and p["slices"] == slices and p["kernel"] == kernel, p
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


def test_noalloc_allocates_no_device_memory():
    # Device free memory (hipMemGetInfo, through torch) is the same before
    # and after a run of split calls, each a different plan; one call per
    # plan first loads the kernels' code objects, whose loading takes
    # device memory of its own.
    ops = []
    for i, (m, n, k, ta, tb, _, _) in enumerate(CASES):
        a, b = operands(m, n, k, ta, tb, seed=51 + i)
        c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        ops.append((a, b, c, ta, tb))
    for a, b, c, ta, tb in ops:
        rt.gemm_noalloc(a, b, c, trans_a=ta, trans_b=tb)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        for a, b, c, ta, tb in ops:
            rt.gemm_noalloc(a, b, c, trans_a=ta, trans_b=tb)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"device free memory moved by {free0 - free1} bytes"


@pytest.mark.parametrize("case", [0, 2, 3], ids=["w4-sum", "128-tree", "skinny"])
def test_noalloc_captured_in_a_graph(case):
    # A split-K noalloc call captured in a HIP graph (after one call outside
    # capture, which resolves the scratch address on this device and loads
    # the kernels), replayed several times with other work and host
    # synchronisations between the replays: every replay equals frisk_gemm
    # with a workspace, bit for bit.
    m, n, k, ta, tb, _, _ = CASES[case]
    a, b = operands(m, n, k, ta, tb, seed=61 + case)
    c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    want = torch.empty_like(c)
    rt.gemm(a, b, want, trans_a=ta, trans_b=tb, workspace=True)
    rt.gemm_noalloc(a, b, c, trans_a=ta, trans_b=tb)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            rt.gemm_noalloc(a, b, c, trans_a=ta, trans_b=tb)
    torch.cuda.current_stream().wait_stream(s)
    other = torch.empty_like(c)
    for r in range(4):
        c.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, want), f"replay {r} differs from frisk_gemm"
        # Eager work on the scratch's plans between replays.
        rt.gemm_noalloc(a, b, other, trans_a=ta, trans_b=tb)
        torch.cuda.synchronize()
        assert torch.equal(other, want)
