"""Execution packets (frisk.export_execution after frisk.infer_layouts) run on
the MI355X through F.execute_packet, checked against the fp64 oracle.

The 64x16 attention case is the reference's fixed-ABI fixture shape
(test/Transforms/attention-layout-fixed-abi.mlir:45-94, Q/K/V 64x16 f16,
scale 0.25, O f32) with the tolerance of run_execution.py:85
(|err| <= 0.002 + 0.002 |ref|)."""
import numpy as np
import pytest
import torch

import frisk_amd as F
from oracle import attention as A
from oracle import gemm as G
from tests import programs as P
from tests.gpu_util import decode, randn

pytestmark = pytest.mark.gpu


def _packet(M, N, D, dtype, threads):
    s, _ = P.attention_tensor_form(M=M, N=N, D=D, dtype=dtype, threads=threads)
    s.module.set_attr("frisk.target", s.builder.get_str_attr("gfx950"))
    F.frisk.infer_layouts(s.module)
    return F.frisk.export_execution(s.module)


@pytest.mark.parametrize("M,N,D,dtype,threads", [(64, 64, 16, "fp16", 128), (128, 64, 64, "bf16", 256),
                                                  (256, 128, 128, "bf16", 512)])
def test_attention_packet(M, N, D, dtype, threads):
    print(f"case packet attention M={M} N={N} D={D} {dtype}", flush=True)
    tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
    g = torch.Generator(device="cuda")
    g.manual_seed(M + N + D)
    q, k, v = ((torch.rand(n, D, generator=g, device="cuda") * 2 - 1).to(tdt) for n in (M, N, N))
    o = torch.full((M, D), float("nan"), dtype=torch.float32, device="cuda")
    # head_dim 16: the packet's contract is not the kernel's (it pads V);
    # the kernel runs the same mathematics on the packet's tensors.
    plan = F.execute_packet(_packet(M, N, D, dtype, threads), [q, k, v, o],
                            allow_layout_mismatch=D < 32)
    torch.cuda.synchronize()
    assert plan["kind"] == "attention" and plan["scale"] == 0.25
    assert plan["layouts_match"] == (D >= 32)
    qd, kd, vd = decode(q), decode(k), decode(v)
    ref = A.attention_fp64(qd[None, None], kd[None, None], vd[None, None], scale=0.25)[0][0, 0]
    err = np.abs(decode(o) - ref)
    if dtype == "fp16":
        # The reference fixture's tolerance (run_execution.py:85).
        assert np.all(err <= 0.002 + 0.002 * np.abs(ref)), err.max()
    else:
        # P enters the PV product in bf16 (unit roundoff u = 2^-8) and the
        # row sum uses the same rounded P, so each normalized weight moves by
        # at most 2u w_j: |err| <= 2^-7 sum_j w_j |v_j| plus f32 noise.
        s = 0.25 * qd @ kd.T
        w = np.exp(s - s.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        assert np.all(err <= 2.0 ** -7 * (w @ np.abs(vd)) + 1e-6), err.max()


@pytest.mark.parametrize("m,k,threads,dtype,variant", [(128, 64, 256, "bf16", (128, 2, 2)),
                                                       (128, 128, 128, "fp16", (128, 1, 2)),
                                                       (256, 64, 256, "bf16", (256, 2, 2)),
                                                       (64, 32, 128, "bf16", None)])
def test_gemm_packet(m, k, threads, dtype, variant):
    print(f"case packet gemm {m}x{m}x{k} threads={threads} {dtype}", flush=True)
    s = F.create_session()
    S = F.MemorySpace.SHARED
    _, entry = s.new_kernel("gemm", [s.memref_type([m, k], dtype, space=S),
                                     s.memref_type([k, m], dtype, space=S),
                                     s.memref_type([m, m], "fp32")])
    c = s.alloc_buffer([m, m], "fp32")
    g = s.create_gemm(entry.get_argument(0), entry.get_argument(1), c, clear_accum=True,
                      legacy_semantics="tensor_v1")
    g.set_attr("frisk.execution_threads", s.builder.get_int64_attr(threads))
    s.builder.create_copy_op(c, entry.get_argument(2), [], [])
    F.frisk.normalize_layout_ir(s.module, "gfx950")
    F.frisk.infer_layouts(s.module)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    a = randn((m, k), 1).to(tdt)
    b = randn((k, m), 2).to(tdt)
    out = torch.full((m, m), float("nan"), dtype=torch.float32, device="cuda")
    # The 64x64 tile on 128 threads has no kernel of its own: it runs on the
    # library's tiling only when the caller allows it.
    plan = F.execute_packet(F.frisk.export_execution(s.module), [a, b, out],
                            allow_layout_mismatch=variant is None)
    torch.cuda.synchronize()
    assert plan["kind"] == "gemm" and plan["variant"] == variant
    assert plan["layouts_match"] == (variant is not None)
    ref = decode(a) @ decode(b)
    assert G.row_scaled_error(decode(out), ref) <= 1e-5


# ---- reduction, fill and copy packets ------------------------------------------------
def _reduce_case(R, C, kind, dtype, dim, threads, init=None):
    from oracle import tileops as T
    from tests.test_packet_tileops import fiber_tree_reference
    dt = {"fp32": "f32", "fp16": "f16"}[dtype]
    tdt = {"f32": torch.float32, "f16": torch.float16}[dt]
    pk = P.exported_packet(P.single_tile_reduce(R, C, kind=kind, dtype=dtype, dim=dim,
                                                threads=threads, init=init))
    rng = np.random.default_rng(R + C + dim + len(kind))
    span = 10 if dt == "f16" else 20
    x = T.round_to(dt, (rng.standard_normal((R, C)) * np.exp2(rng.integers(-span, span + 1, (R, C))))
                   .astype(np.float32))
    n = R if dim == 1 else C
    y = torch.full((n,), 9.0, dtype=tdt, device="cuda")
    plan = F.execute_packet(pk, [torch.from_numpy(x).to(tdt).cuda(), y])
    torch.cuda.synchronize()
    want = fiber_tree_reference(pk, x, kind, dt)
    if init is not None:
        want = T.combine(T.KINDS[kind], dt, np.full(n, init, dtype=np.float32), want)
    got = y.float().cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].astype(np.float32).view(np.uint32))
    return plan


@pytest.mark.parametrize("dim", [1, 0])
@pytest.mark.parametrize("kind", ["add", "max"])
@pytest.mark.parametrize("dtype", ["fp32", "fp16"])
@pytest.mark.parametrize("shape,threads", [((64, 64), 128), ((32, 16), 64), ((128, 32), 256)])
def test_reduce_packet_matches_its_fibers(shape, threads, dtype, kind, dim):
    """The packet's sums follow its fibers' tree, including the permuted row
    order of the column sums, bit for bit."""
    print(f"case reduce packet {shape} threads={threads} {dtype} {kind} dim={dim}", flush=True)
    _reduce_case(*shape, kind, dtype, dim, threads)


@pytest.mark.parametrize("kind,init", [("max", float("-inf")), ("add", 0.5), ("min", 3.0)])
def test_merge_reduce_packet(kind, init):
    print(f"case merge packet {kind} {init}", flush=True)
    plan = _reduce_case(64, 64, kind, "fp32", 1, 128, init=init)
    assert plan["init"] == init


def test_fill_and_copy_packets_run():
    print("case fill/copy packets", flush=True)
    y = torch.zeros(64, 64, device="cuda")
    F.execute_packet(P.exported_packet(P.single_tile_fill(64, 64, value=-2.25)), [y])
    x = torch.randn(64, 64, device="cuda")
    z = torch.zeros(64, 64, device="cuda")
    F.execute_packet(P.exported_packet(P.single_tile_copy(64, 64)), [x, z])
    torch.cuda.synchronize()
    assert torch.equal(y, torch.full_like(y, -2.25)) and torch.equal(x, z)
