"""The C-ABI's stream and threading contract on the GPU (include/frisk_hip.h:
calls are stream-ordered on the caller's hipStream_t and reentrant): work
passed a non-default stream runs on that stream, and two host threads
launching on their own streams at once both get correct results."""
import threading

import torch
import pytest

from frisk_amd import runtime as rt
from tests.gpu_util import randn

pytestmark = pytest.mark.gpu


def test_launches_go_to_the_callers_stream():
    # A chain of large GEMMs on a side stream: right after the launches the
    # side stream is still busy while torch's current stream has nothing
    # queued, so the C-ABI enqueued on the stream it was given.
    s = torch.cuda.Stream()
    a = randn((8192, 8192), 1).to(torch.bfloat16)
    b = randn((8192, 8192), 2).to(torch.bfloat16)
    cs = [torch.empty(8192, 8192, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    for i in range(20):
        rt.gemm(a, b, cs[i % 2], trans_b=True, stream=s)
    assert not s.query(), "side stream idle right after 20 launches of 8192^3"
    assert torch.cuda.current_stream().query(), "work landed on the current stream"
    s.synchronize()
    want = torch.empty_like(cs[0])
    rt.gemm(a, b, want, trans_b=True)
    torch.cuda.synchronize()
    assert torch.equal(cs[1], want)


def test_two_host_threads_launch_concurrently():
    # Each thread owns a stream and launches GEMMs and attention forwards on
    # it in a loop; every output equals the same call made alone.
    n = 2
    inputs = []
    for t in range(n):
        a = randn((1024 + 256 * t, 2048), 10 + t).to(torch.bfloat16)
        b = randn((1536, 2048), 20 + t).to(torch.bfloat16)
        q, k, v = (randn((2, 8, 1024, 128), 30 + 3 * t + i).to(torch.bfloat16) for i in range(3))
        inputs.append((a, b, q, k, v))
    want = []
    for a, b, q, k, v in inputs:
        c = torch.empty(a.shape[0], b.shape[0], dtype=torch.bfloat16, device="cuda")
        o = torch.empty_like(q)
        rt.gemm(a, b, c, trans_b=True)
        rt.attn_fwd(q, k, v, o, causal=True)
        want.append((c, o))
    torch.cuda.synchronize()
    outs = [None] * n
    errors = []
    start = threading.Barrier(n)

    def work(t):
        try:
            s = torch.cuda.Stream()
            a, b, q, k, v = inputs[t]
            c = torch.empty(a.shape[0], b.shape[0], dtype=torch.bfloat16, device="cuda")
            o = torch.empty_like(q)
            start.wait()
            for _ in range(25):
                rt.gemm(a, b, c, trans_b=True, stream=s)
                rt.attn_fwd(q, k, v, o, causal=True, stream=s)
            s.synchronize()
            outs[t] = (c, o)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(n)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not errors, errors
    for t in range(n):
        assert torch.equal(outs[t][0], want[t][0]) and torch.equal(outs[t][1], want[t][1])
