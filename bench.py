#!/usr/bin/env python3
"""Benchmark of the GEMM + attention hot path on one MI355X.

A step is one launch of the headline kernel over one batch of synthetic,
HBM-resident input: the bf16 GEMM C[4096, 4096] = A[4096, 4096] . B^T with
B stored [N, K] (A and B ~ N(0, 1), f32 accumulation, bf16 output), the
"bf16 4096^3" of BASELINE.json's metric.  `value` is its TFLOP/s
(2*M*N*K per launch).  The same JSON line carries the other workloads the
metric names, each timed the same way (--settle seconds of untimed launches
to bring the GPU to its steady clock, W warm-up launches, then K timed
launches between device synchronisations): fp16 4096^3 NT,
fp8-e4m3 4096x8192x8192 with per-tensor scales, int8 4096^3,
and the flash-attention forward at b4 h32 s4096 d128 bf16, non-causal and
causal (configs[4]; causal FLOPs counted as half).  `projection_sweep` holds
the 12 bf16 projection GEMMs of configs[2], each against its own roofline
(HBM or MFMA), with hipBLASLt's time on the same tensors beside it.  The HBM-bound tile ops
on either side of them (frisk_reduce, frisk_copy with an f32 -> bf16
conversion, frisk_fill) are reported in GB/s of algorithmic traffic (each
input byte read once, each output byte written once) against the 8 TB/s
HBM peak.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --only NAME[,NAME...] --steps K   (for rocprofv3)
       python bench.py --trace-summary KERNEL_TRACE.csv --steps K
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK = {"bf16": 2500.0, "f16": 2500.0, "fp8": 5000.0, "int8": 5000.0,
        "f32": 157.3}  # dense TFLOP/s (TOP/s)
REF_FIXED_TILE_US = {"single": 21.584, "graph": 6.5386}  # the reference's published H100 figures
HBM_PEAK_GBS = 8000.0
PEAK_MHZ = 2400.0  # shader clock of the published MFMA peaks
SETTLE_S = 0.25  # untimed load before each workload's warm-up, see time_launches


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--only", default=None,
                   help="run only these workloads (comma-separated), for profilers")
    p.add_argument("--trace-summary", default=None, metavar="CSV",
                   help="summarise a rocprofv3 kernel-trace CSV of a --only run and exit")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--settle", type=float, default=SETTLE_S,
                   help="seconds of untimed load before each workload's warm-up")
    return p.parse_args()


def make_workloads(torch, rt):
    """name -> (dtype label, flops per launch, setup() -> launch callable)."""
    dev = "cuda"

    def gen(seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        return g

    def gemm(m, n, k, kind, trans_a=False, trans_b=True):
        # A stored [M, K] ([K, M] with trans_a), B stored [N, K] ([K, N]
        # without trans_b).
        a_shape = (k, m) if trans_a else (m, k)
        b_shape = (n, k) if trans_b else (k, n)

        def setup():
            if kind == "int8":
                a = torch.randint(-127, 128, a_shape, generator=gen(1), device=dev, dtype=torch.int8)
                b = torch.randint(-127, 128, b_shape, generator=gen(2), device=dev, dtype=torch.int8)
                c = torch.empty(m, n, dtype=torch.int32, device=dev)
                return lambda: rt.gemm(a, b, c, trans_a=trans_a, trans_b=trans_b)
            if kind == "fp8":
                a = torch.randn(a_shape, generator=gen(1), device=dev)
                b = torch.randn(b_shape, generator=gen(2), device=dev)
                sa, sb = 448.0 / float(a.abs().max()), 448.0 / float(b.abs().max())
                a8, b8 = (a * sa).to(torch.float8_e4m3fn), (b * sb).to(torch.float8_e4m3fn)
                del a, b
                c = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
                return lambda: rt.gemm(a8, b8, c, trans_a=trans_a, trans_b=trans_b,
                                       scale_a=1 / sa, scale_b=1 / sb)
            dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[kind]
            a = torch.randn(a_shape, generator=gen(1), device=dev).to(dt)
            b = torch.randn(b_shape, generator=gen(2), device=dev).to(dt)
            c = torch.empty(m, n, dtype=dt, device=dev)
            return lambda: rt.gemm(a, b, c, trans_a=trans_a, trans_b=trans_b)
        return setup

    def attn(causal, k_transposed=False):
        def setup():
            shape = (4, 32, 4096, 128)
            q = torch.randn(shape, generator=gen(5), device=dev).to(torch.bfloat16)
            k = torch.randn(shape, generator=gen(6), device=dev).to(torch.bfloat16)
            v = torch.randn(shape, generator=gen(7), device=dev).to(torch.bfloat16)
            o = torch.empty_like(q)
            if k_transposed:  # K stored [B, H, D, S], read in place
                k = k.transpose(-1, -2).contiguous()
            return lambda: rt.attn_fwd(q, k, v, o, causal=causal, sm_scale=128 ** -0.5,
                                       k_transposed=k_transposed)
        return setup

    def library_gemm(m, n, k):
        def setup():
            a = torch.randn(m, k, generator=gen(1), device=dev).to(torch.bfloat16)
            b = torch.randn(n, k, generator=gen(2), device=dev).to(torch.bfloat16)
            return lambda: torch.matmul(a, b.t())
        return setup

    def library_gemm_fp8(m, n, k):
        # torch._scaled_mm (hipBLASLt) on the fp8 workload's operands and scales.
        def setup():
            a = torch.randn(m, k, generator=gen(1), device=dev)
            b = torch.randn(n, k, generator=gen(2), device=dev)
            sa, sb = 448.0 / float(a.abs().max()), 448.0 / float(b.abs().max())
            a8, b8 = (a * sa).to(torch.float8_e4m3fn), (b * sb).to(torch.float8_e4m3fn)
            del a, b
            ia = torch.tensor(1 / sa, device=dev)
            ib = torch.tensor(1 / sb, device=dev)
            return lambda: torch._scaled_mm(a8, b8.t(), scale_a=ia, scale_b=ib,
                                            out_dtype=torch.bfloat16)
        return setup

    def copy(nbytes):
        def setup():
            src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
            dst = torch.empty_like(src)
            return lambda: dst.copy_(src)
        return setup

    def attn_d64():
        def setup():
            shape = (2, 32, 1025, 64)
            q = (torch.rand(shape, generator=gen(8), device=dev) * 2 - 1).half()
            k = (torch.rand(shape, generator=gen(9), device=dev) * 2 - 1).half()
            v = (torch.rand(shape, generator=gen(10), device=dev) * 2 - 1).half()
            o = torch.empty(shape, dtype=torch.float32, device=dev)
            return lambda: rt.attn_fwd(q, k, v, o, causal=False, sm_scale=0.125)
        return setup

    def reduce(rows, cols, axis, kind):
        def setup():
            x = torch.randn(rows, cols, generator=gen(11), device=dev)
            out = torch.empty(rows if axis == 1 else cols, device=dev)
            ws = torch.empty(max(rt.reduce_workspace_bytes(x, out, kind, axis=axis), 16),
                             dtype=torch.uint8, device=dev)
            return lambda: rt.reduce(x, out, kind, axis=axis, workspace=ws)
        return setup

    def cast(rows, cols):
        def setup():
            x = torch.randn(rows, cols, generator=gen(12), device=dev)
            y = torch.empty(rows, cols, dtype=torch.bfloat16, device=dev)
            return lambda: rt.copy(x, y)
        return setup

    def fill(rows, cols):
        def setup():
            y = torch.empty(rows, cols, dtype=torch.bfloat16, device=dev)
            return lambda: rt.fill(y, 0.5)
        return setup

    fa = 4.0 * 4 * 32 * 4096 * 4096 * 128
    return {
        "gemm_bf16_4096": ("bf16", 2.0 * 4096 ** 3, gemm(4096, 4096, 4096, "bf16")),
        # The other storage orders of the headline GEMM: NN is the builder's
        # default (transA = transB = False) and the reference's GEMM tile
        # program's B [K, N] (tmp/ir.mlir:2-16).
        "gemm_bf16_4096_nn": ("bf16", 2.0 * 4096 ** 3, gemm(4096, 4096, 4096, "bf16", False, False)),
        "gemm_bf16_4096_tn": ("bf16", 2.0 * 4096 ** 3, gemm(4096, 4096, 4096, "bf16", True, True)),
        "gemm_bf16_4096_tt": ("bf16", 2.0 * 4096 ** 3, gemm(4096, 4096, 4096, "bf16", True, False)),
        "gemm_f16_4096_nt": ("f16", 2.0 * 4096 ** 3, gemm(4096, 4096, 4096, "f16")),
        "gemm_fp8_4096x8192x8192": ("fp8", 2.0 * 4096 * 8192 * 8192,
                                    gemm(4096, 8192, 8192, "fp8")),
        "gemm_int8_4096": ("int8", 2.0 * 4096 ** 3, gemm(4096, 4096, 4096, "int8")),
        # fp32 on v_mfma_f32_32x32x2_f32: the reference's GEMM tile program
        # (fp32 1024^3, B [K, N], tmp/ir.mlir:2-16) and configs[0] (512^3).
        "gemm_f32_1024_nn": ("f32", 2.0 * 1024 ** 3, gemm(1024, 1024, 1024, "f32", False, False)),
        "gemm_f32_512_nn": ("f32", 2.0 * 512 ** 3, gemm(512, 512, 512, "f32", False, False)),
        "fa_fwd_b4h32s4096d128": ("bf16", fa, attn(False)),
        "fa_fwd_b4h32s4096d128_causal": ("bf16", fa / 2, attn(True)),
        # K stored [B, H, D, S]: the reference's FA tile program layout
        # (tmp/ir.mlir:89-92), read in place.
        "fa_fwd_b4h32s4096d128_kt": ("bf16", fa, attn(False, True)),
        "fa_fwd_b4h32s4096d128_kt_causal": ("bf16", fa / 2, attn(True, True)),
        "fa_fwd_d64_b2h32s1025_f16_f32out": ("f16", 4.0 * 2 * 32 * 1025 * 1025 * 64, attn_d64()),
        # HBM-bound tile ops: second entry = algorithmic bytes per launch.
        "reduce_sum_f32_32768x4096_rows": ("hbm", 32768 * 4096 * 4 + 32768 * 4,
                                           reduce(32768, 4096, 1, "sum")),
        "reduce_max_f32_8192x16384_cols": ("hbm", 8192 * 16384 * 4 + 16384 * 4,
                                           reduce(8192, 16384, 0, "max")),
        "copy_f32_to_bf16_16384x8192": ("hbm", 16384 * 8192 * (4 + 2), cast(16384, 8192)),
        "fill_bf16_16384x16384": ("hbm", 16384 * 16384 * 2, fill(16384, 16384)),
        # Calibration only (--only): a plain 256 MiB device copy, whose
        # FETCH_SIZE / WRITE_SIZE per dispatch scale the HBM counters.
        "copy_256mib": ("bytes", 0.0, copy(256 << 20)),
        # Comparison only (--only): hipBLASLt (torch.matmul) on the headline
        # GEMM's operands, for counter passes beside gemm_bf16_4096.
        "hipblaslt_bf16_4096": ("ref", 2.0 * 4096 ** 3, library_gemm(4096, 4096, 4096)),
        "hipblaslt_fp8_4096x8192x8192": ("ref", 2.0 * 4096 * 8192 * 8192,
                                         library_gemm_fp8(4096, 8192, 8192)),
    }


def time_launches(torch, fn, steps, warmup, settle_s=SETTLE_S, counts=None):
    # An idle MI355X takes about 50 ms of load to reach its steady clock
    # (measured: the first 25 ms of 4096^3 GEMMs run at 1090 TFLOP/s, every
    # later window at 1230 for seconds).  The untimed settle runs the workload
    # for settle_s before the W warm-up launches, so that the K timed launches
    # see the clock a sustained workload sees.
    t0 = time.perf_counter()
    settled = 0
    while time.perf_counter() - t0 < settle_s:
        for _ in range(8):
            fn()
        settled += 8
        torch.cuda.synchronize()
    if counts is not None:
        counts.update(settle=settled, warmup=warmup, timed=steps)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per launch


def launch_percentiles(torch, fn, n=50):
    """p10 / p50 / p90 of n individually event-timed launches (ms)."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in ev)
    pick = lambda q: t[min(n - 1, int(q * (n - 1) + 0.5))]
    return {"p10": round(pick(0.1), 6), "p50": round(pick(0.5), 6), "p90": round(pick(0.9), 6)}


def provenance(torch):
    """What was measured: hashes of the kernel sources and of the built
    library, the git commit recorded at build time, and the GPU."""
    from frisk_amd.build import source_digest
    lib = ROOT / "frisk_amd" / "libfrisk_hip.so"
    info = {}
    bi = ROOT / "frisk_amd" / "BUILD_INFO.json"
    if bi.exists():
        info = json.loads(bi.read_text())
    props = torch.cuda.get_device_properties(0)
    gpu = {"name": props.name, "arch": getattr(props, "gcnArchName", None),
           "cus": props.multi_processor_count, "mem_gib": round(props.total_memory / 2 ** 30, 1)}
    uuid = getattr(props, "uuid", None)
    if uuid is not None:
        gpu["uuid"] = str(uuid)
    return {"source_sha256_16": source_digest(),
            "library_sha256_16": hashlib.sha256(lib.read_bytes()).hexdigest()[:16] if lib.exists() else None,
            "git_commit": info.get("git_commit"), "built_source_sha256_16": info.get("source_sha256_16"),
            "gpu": gpu, "torch": torch.__version__, "hip": torch.version.hip}


def projection_sweep(torch, rt, steps, warmup, settle_s):
    """Y[M, N] = X[M, K] . W[N, K]^T in bf16 for (N, K) in
    {(4096, 4096), (14336, 4096), (4096, 14336)} and M in {16, 128, 1024,
    8192}, W ~ N(0, 0.02), X ~ N(0, 1).  Each shape is timed like the other
    workloads, with the split-K workspace allocated before timing, and
    reported against its own roofline: HBM when its FLOP per algorithmic
    byte (M.K + N.K + M.N, 2 bytes each) is below the ridge (2.5 PFLOP/s /
    8 TB/s), MFMA otherwise.  Consecutive launches cycle through enough
    copies of X, W and Y (>= 600 MB together) that no launch finds its
    operands in the 256 MB last-level cache.  torch.matmul (hipBLASLt) on
    the same tensors, cycled the same way, is timed beside it."""
    g = torch.Generator(device="cuda")
    out = {}
    ridge = PEAK["bf16"] * 1e12 / (HBM_PEAK_GBS * 1e9)
    for n, k in ((4096, 4096), (14336, 4096), (4096, 14336)):
        for m in (16, 128, 1024, 8192):
            per_copy = 2 * (m * k + n * k + m * n)
            copies = max(1, -(-600_000_000 // per_copy))
            g.manual_seed(3)
            w0 = (torch.randn(n, k, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
            g.manual_seed(4 + m)
            x0 = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16)
            ops = [(x0.clone(), w0.clone(), torch.empty(m, n, dtype=torch.bfloat16, device="cuda"))
                   for _ in range(copies)]
            del w0, x0
            need = rt.gemm_workspace_bytes(*ops[0], trans_b=True)
            ws = torch.empty(need, dtype=torch.uint8, device="cuda") if need > 0 else False
            turn = [0]

            def ours():
                x, w, y = ops[turn[0] % copies]
                turn[0] += 1
                rt.gemm(x, w, y, trans_b=True, workspace=ws)

            def blas():
                x, w, _ = ops[turn[0] % copies]
                turn[0] += 1
                torch.matmul(x, w.t())

            ms = time_launches(torch, ours, steps, warmup, settle_s)
            ms_blas = time_launches(torch, blas, steps, warmup, settle_s)
            flops, nbytes = 2.0 * m * n * k, 2.0 * (m * k + n * k + m * n)
            tf, gbs = flops / ms / 1e9, nbytes / ms / 1e6
            bound = "hbm" if flops / nbytes < ridge else "mfma"
            frac = gbs / HBM_PEAK_GBS if bound == "hbm" else tf / PEAK["bf16"]
            print(f"bench: projection m{m} n{n} k{k} {ms * 1e3:.2f} us", file=sys.stderr, flush=True)
            out[f"m{m}_n{n}_k{k}"] = {"us": round(ms * 1e3, 2), "tflops": round(tf, 1),
                                       "gbs": round(gbs, 1), "bound": bound,
                                       "frac": round(frac, 4), "split_k": need > 0,
                                       "operand_copies": copies,
                                       "hipblaslt_us": round(ms_blas * 1e3, 2)}
            del ops, ws
            torch.cuda.empty_cache()
    return out


def fixed_tile_latency(torch, rt):
    """The reference's 64x16 attention tile: single-launch and graph-amortized
    per-launch time in microseconds (see module docstring)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    q, k, v = ((torch.rand(1, 1, 64, 16, generator=g, device="cuda") * 2 - 1).half() for _ in range(3))
    o = torch.empty(1, 1, 64, 16, dtype=torch.float32, device="cuda")

    def launch():
        rt.attn_fwd(q, k, v, o, sm_scale=0.25)

    for _ in range(20):
        launch()
    torch.cuda.synchronize()
    single = []
    for _ in range(20):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        launch()
        b.record()
        b.synchronize()
        single.append(a.elapsed_time(b) * 1e3)
    per_graph = 100
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            launch()
    graph.replay()
    torch.cuda.synchronize()
    replays = []
    for _ in range(20):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        replays.append(a.elapsed_time(b) * 1e3 / per_graph)
    single.sort()
    replays.sort()
    return {"single_us_median": round(single[len(single) // 2], 3),
            "graph_us_median": round(replays[len(replays) // 2], 3),
            "reference_h100_us": REF_FIXED_TILE_US,
            "speedup_vs_reference": {"single": round(REF_FIXED_TILE_US["single"] / single[len(single) // 2], 2),
                                     "graph": round(REF_FIXED_TILE_US["graph"] / replays[len(replays) // 2], 2)}}


def _repeat(fn, min_seconds, max_reps):
    """Runs fn until min_seconds of wall time have passed (at most max_reps
    times); returns (repetitions, seconds)."""
    reps = 0
    t0 = time.perf_counter()
    while reps < max_reps:
        fn()
        reps += 1
        if time.perf_counter() - t0 >= min_seconds:
            break
    return reps, time.perf_counter() - t0


def cpu_baseline(torch, min_seconds=10.0, max_passes=8):
    """fp64 C oracle (oracle/oracle.c) on bounded samples of the headline
    workloads, on this host's cores.  Top level: the bf16 4096^3 GEMM
    (inputs decoded exactly from bf16) in blocks of 512 output rows, whole
    passes over the 4096 rows repeated until at least `min_seconds` of wall
    time (at most `max_passes`), on all CPU threads of this process.  `legs`:
    the same GEMM on one core (64 output rows), and the attention forward of
    configs[4] (b4 h32 s4096 d128) for 128 query rows of one head on all
    threads and 16 rows on one core (4 * rows * s * d FLOPs: QK^T and PV).
    `manifest` names the seed and shapes of every sample and carries a
    SHA-256 over the sample inputs (as bf16 bytes) and the oracle's C
    source, so two baselines can be checked to have timed the same work;
    `cpu_model` is the host's CPU."""
    import numpy as np
    from oracle import native
    native.load()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or native.max_threads()
    m, n, k, blk = 4096, 4096, 4096, 512
    g = torch.Generator()
    g.manual_seed(1)
    digest = hashlib.sha256((ROOT / "oracle" / "oracle.c").read_bytes())

    def sample(rows, cols):
        t = torch.randn(rows, cols, generator=g).to(torch.bfloat16)
        digest.update(t.view(torch.int16).numpy().tobytes())
        return t.double().numpy()

    a = sample(m, k)
    b = sample(n, k)
    native.gemm_f64(a[:8], b, trans_b=True, threads=threads)  # warm up threads

    def gemm_pass():
        for r0 in range(0, m, blk):
            native.gemm_f64(a[r0:r0 + blk], b, trans_b=True, threads=threads)

    passes, dt = _repeat(gemm_pass, min_seconds, max_passes)
    rows = passes * m
    out = {"value": round(2.0 * rows * n * k / dt / 1e12, 6), "unit": "TFLOP/s",
           "cores": threads, "kind": "port",
           "sample": f"{passes} full pass(es) over the 4096^3 GEMM in 512-row blocks "
                     f"(fp64 oracle/oracle.c, {dt:.1f} s wall)"}
    legs = {}
    reps, dt = _repeat(lambda: native.gemm_f64(a[:64], b, trans_b=True, threads=1), 2.0, 50)
    legs["gemm_bf16_4096_single_core"] = {
        "value": round(2.0 * 64 * reps * n * k / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
        "kind": "port", "sample": f"{reps} x 64 output rows of the 4096^3 GEMM ({dt:.1f} s)"}
    s_len, d = 4096, 128
    q = sample(s_len, d)
    kk = sample(s_len, d)
    v = sample(s_len, d)
    for name, nrows, nthreads, secs in (("fa_fwd_b4h32s4096d128", 128, threads, 4.0),
                                        ("fa_fwd_b4h32s4096d128_single_core", 16, 1, 2.0)):
        rows_idx = np.arange(0, s_len, s_len // nrows, dtype=np.int64)[:nrows]
        reps, dt = _repeat(lambda: native.attn_rows_f64(q, kk, v, rows_idx, scale=d ** -0.5,
                                                         threads=nthreads), secs, 100000)
        legs[name] = {"value": round(4.0 * nrows * reps * s_len * d / dt / 1e12, 6),
                      "unit": "TFLOP/s", "cores": nthreads, "kind": "port",
                      "sample": f"{reps} x {nrows} query rows of one head, s=4096 d=128, "
                                f"non-causal (fp64 oracle_attn_rows_f64, {dt:.1f} s)"}
    out["legs"] = legs
    out["cpu_model"] = _cpu_model()
    out["manifest"] = {
        "seed": 1, "draws": "torch.randn (CPU generator) in order A[4096,4096], B[4096,4096], "
                            "Q[4096,128], K[4096,128], V[4096,128], each rounded to bf16",
        "gemm": [m, n, k], "attn": [s_len, d], "oracle": "oracle/oracle.c",
        "sha256_16": digest.hexdigest()[:16]}
    return out


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or None


def traffic_from_profile(name):
    """HBM bytes per launch recorded from rocprofv3 FETCH_SIZE/WRITE_SIZE
    passes (profiles/hbm_traffic.txt, one JSON object per line)."""
    path = ROOT / "profiles" / "hbm_traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        line = line.strip()
        if line.startswith("{"):
            rec = json.loads(line)
            if rec.get("kernel_workload") == name:
                return rec.get("traffic_bytes")
    return None


def _kernel_short(name):
    """A kernel's name without its parameter list, `void` and namespace, and
    with the enum casts of its template arguments dropped."""
    cut = name.find(">(")
    base = name[:cut + 1] if cut >= 0 else name.split("(")[0]
    return base.replace("void ", "").replace("frisk::", "").replace("(Elt)", "").strip()


def trace_summary(path, steps):
    """Per-kernel durations from a rocprofv3 kernel trace, its CSV (`-f csv`)
    or its results database (`*_results.db`, the default format): dispatch
    count, average, minimum and maximum over every dispatch (settle and
    warm-up included) and over the last `steps` dispatches of that kernel
    and grid, which in a `--only` run are the timed launches.  Returns a list
    of dicts, the longest kernels first."""
    rows = {}
    if str(path).endswith(".db"):
        import sqlite3
        con = sqlite3.connect(path)
        for name, start, end, gx, gy, gz, wx, wy, wz in con.execute(
                "select name, start, end, grid_x, grid_y, grid_z, workgroup_x, workgroup_y, "
                "workgroup_z from kernels"):
            grid = (gx // max(1, wx), gy // max(1, wy), gz // max(1, wz))
            rows.setdefault((name, grid), []).append((int(start), (int(end) - int(start)) / 1e3))
    else:
        import csv
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                grid = tuple(int(r[f"Grid_Size_{a}"]) // max(1, int(r[f"Workgroup_Size_{a}"]))
                             for a in "XYZ")
                key = (r["Kernel_Name"], grid)
                rows.setdefault(key, []).append(
                    (int(r["Start_Timestamp"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    out = []
    for (name, grid), d in rows.items():
        d.sort()
        us = [x[1] for x in d]
        last = us[-steps:]
        out.append({"kernel": _kernel_short(name), "grid": grid, "calls": len(us),
                    "avg_us": sum(us) / len(us), "min_us": min(us), "max_us": max(us),
                    "timed_calls": len(last),
                    "timed_avg_us": sum(last) / len(last), "timed_min_us": min(last),
                    "timed_max_us": max(last),
                    "timed_span_us": (d[-1][0] - d[-len(last)][0]) / 1e3 + d[-1][1]})
    out.sort(key=lambda r: -r["timed_avg_us"])
    return out


def main():
    args = parse()
    if args.trace_summary:
        for r in trace_summary(args.trace_summary, args.steps):
            print(json.dumps(r))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "GEMM and attention shard across GPUs without exchange",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from frisk_amd import runtime as rt
    from frisk_amd.clock import sustained_clock
    rt.load()
    torch.cuda.set_device(0)
    work = make_workloads(torch, rt)
    if args.only == "fixed_tile_64x16":
        print(json.dumps({"workload": args.only, **fixed_tile_latency(torch, rt)}), flush=True)
        return
    if args.only:
        # Each workload: settle, warm-up, then the K timed launches, and
        # nothing after them, so the last K dispatches of its kernels in a
        # kernel trace are the timed ones (--trace-summary).
        for name in args.only.split(","):
            label, flops, setup = work[name]
            fn = setup()
            counts = {}
            ms = time_launches(torch, fn, args.steps, args.warmup, args.settle, counts)
            rate = {"gbs": flops / ms / 1e6} if label == "hbm" else {"tflops": flops / ms / 1e9}
            print(json.dumps({"workload": name, "ms": ms, **rate, "launches": counts}), flush=True)
            del fn
            torch.cuda.empty_cache()
        return

    results = {}
    for name, (label, flops, setup) in work.items():
        if label in ("bytes", "ref"):
            continue
        fn = setup()
        steps = args.steps
        ms = time_launches(torch, fn, steps, args.warmup, args.settle)
        if label == "hbm":
            gbs = flops / ms / 1e6
            results[name] = {"bytes": flops, "ms": round(ms, 6), "gbs": round(gbs, 1),
                             "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                             "traffic": traffic_from_profile(name)}
        else:
            tf = flops / ms / 1e9
            mhz = sustained_clock(torch, fn)
            results[name] = {"dtype": label, "ms": round(ms, 6), "tflops": round(tf, 2),
                             "frac_peak": round(tf / PEAK[label], 4),
                             "sclk_mhz": mhz,
                             "frac_peak_at_sclk": round(tf / (PEAK[label] * mhz / PEAK_MHZ), 4) if mhz else None,
                             "launch_ms": launch_percentiles(torch, fn),
                             "traffic": traffic_from_profile(name)}
        print(f"bench: {name} {ms * 1e3:.2f} us", file=sys.stderr, flush=True)
        del fn
        torch.cuda.empty_cache()

    head = results["gemm_bf16_4096"]
    flops = 2.0 * 4096 ** 3
    traffic = traffic_from_profile("gemm_bf16_4096")
    line = {
        "metric": "GEMM TFLOP/s & % MFMA peak (bf16/fp8 4096^3); FA-fwd TFLOP/s at s=4096",
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": args.settle,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1), HBM-resident before timing)",
        "config": {"workload": "bf16 GEMM M=N=K=4096, A [M,K] row-major, B [N,K] (NT), "
                               "f32 accumulate, bf16 out; one launch per step",
                   "m": 4096, "n": 4096, "k": 4096, "layout": "NT"},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": PEAK["bf16"],
                     "unit": "TFLOP/s", "frac": round(head["tflops"] / PEAK["bf16"], 4),
                     "traffic": traffic, "sclk_mhz": head["sclk_mhz"],
                     "frac_at_sclk": head["frac_peak_at_sclk"]},
        "provenance": provenance(torch),
        "workloads": results,
        "projection_sweep": projection_sweep(torch, rt, args.steps, args.warmup, 0.1),
        "fixed_tile_64x16": fixed_tile_latency(torch, rt),
    }
    if not args.no_cpu:
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
