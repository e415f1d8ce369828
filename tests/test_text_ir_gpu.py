"""Textual IR run on the GPU: a tile program printed, parsed back
(F.parse_module, frisk_amd/ir/parse.cpp) and executed through F.execute, and
an attention program taken through the frisk-opt driver
(`python -m frisk_amd.opt ... --frisk-infer-layouts --frisk-export-execution`,
the reference's tools/frisk-opt/frisk-opt.cpp feeding
benchmark/layout/execution/run_execution.py:23) whose packet runs through
F.execute_packet.  Results are checked against the fp64 oracle with the same
tolerances as the builder-made programs."""
import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import frisk_amd as F
from oracle import attention as A
from oracle import gemm as G
from tests import programs as P
from tests.gpu_util import decode, randn

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]


def parsed(module):
    text = F._ir().frisk.print_module(module)
    m = F.parse_module(text)
    assert m.verify(), m.verify_diagnostic()
    return m


@pytest.mark.parametrize("ta,tb", [(False, False), (True, True)], ids=["nn", "tt"])
def test_parsed_tiled_gemm_executes(ta, tb):
    M, N, K = 512, 384, 640
    print(f"text-ir gemm ta={ta} tb={tb}", flush=True)
    s, _ = P.tiled_gemm(M, N, K, BM=128, BN=128, BK=64, dtype="bf16", out="bf16",
                        trans_a=ta, trans_b=tb)
    m = parsed(s.module)
    a = randn((K, M) if ta else (M, K), 11).to(torch.bfloat16)
    b = randn((N, K) if tb else (K, N), 12).to(torch.bfloat16)
    c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    F.execute(m, "matmul", [a, b, c])
    torch.cuda.synchronize()
    A_ = decode(a).T if ta else decode(a)
    B_ = decode(b).T if tb else decode(b)
    assert G.row_scaled_error(decode(c), A_ @ B_) <= 1e-2


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_parsed_attention_executes(causal):
    Bt, H, S, D = 1, 4, 512, 128
    print(f"text-ir attention causal={causal}", flush=True)
    s, _ = P.attention(Bt, H, S, D)
    m = parsed(s.module)
    q, k, v = (randn((Bt, H, S, D), 30 + i).to(torch.bfloat16) for i in range(3))
    o = torch.full_like(q, float("nan"))
    F.execute(m, "attention", [q, k, v, o], causal=causal)
    torch.cuda.synchronize()
    ro, _ = A.attention_fp64(decode(q), decode(k), decode(v), causal=causal)
    assert G.row_scaled_error(decode(o).reshape(-1, D), ro.reshape(-1, D)) <= 1e-2


def test_frisk_opt_packet_executes(tmp_path):
    # The fixed-ABI attention tile (64x16 f16, scale 0.25, f32 O): printed,
    # then normalized, inferred and exported by the frisk-opt driver in a
    # child process, the packet JSON read back and executed.
    s, _ = P.attention_tensor_form(M=64, N=64, D=16, dtype="fp16", threads=128)
    src = tmp_path / "attn.mlir"
    src.write_text(F._ir().frisk.print_module(s.module))
    out = tmp_path / "packet.json"
    r = subprocess.run([sys.executable, "-m", "frisk_amd.opt", str(src),
                        "--frisk-infer-layouts=target=gfx950",
                        f"--frisk-export-execution=output={out}"],
                       cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    packet = json.loads(out.read_text())
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    q, k, v = ((torch.rand(64, 16, generator=g, device="cuda") * 2 - 1).half() for _ in range(3))
    o = torch.full((64, 16), float("nan"), dtype=torch.float32, device="cuda")
    # head_dim 16 is not the attention kernel's contract (the kernel pads V).
    plan = F.execute_packet(packet, [q, k, v, o], allow_layout_mismatch=True)
    torch.cuda.synchronize()
    assert plan["kind"] == "attention"
    qd, kd, vd = decode(q), decode(k), decode(v)
    ref = A.attention_fp64(qd[None, None], kd[None, None], vd[None, None], scale=0.25)[0][0, 0]
    # The reference fixture's tolerance (run_execution.py:85).
    assert np.all(np.abs(decode(o) - ref) <= 0.002 + 0.002 * np.abs(ref))
