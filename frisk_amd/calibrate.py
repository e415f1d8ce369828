"""Calibration of the layout solver's cost weights against kernel times.

Layout inference (frisk_amd/ir/infer.cpp) scores a candidate assignment as
sum_f w_f x_f over named features x_f (MFMA issue cycles, LDS read/write
cycles, fragment LDS read instructions, 128-byte global lines, VALU / transcendental / cross-lane issue,
conversion bytes, barriers).  The default profile `cdna4-layout-v1` takes w
from hardware rates.  This module fits w to what the compiled kernels take on
the MI355X, and writes the result as a cost profile that inference loads
(`F.frisk.infer_layouts(module, cost_profile=text)`, or
`python -m frisk_amd.opt ... --frisk-infer-layouts=cost-profile=NAME`).
The reference's counterpart is its calibrated SM90 model: frozen integer
coefficients over its own feature set, loaded from a profile file whose
SHA-256 names the model
(lib/Dialect/Frisk/Target/SM90/SM90CalibratedCostModel.cpp:26-35,276-292).

The sweep.  Every row is one kernel launch the C-ABI makes:

  * GEMM: each kernel variant (256x256 tile with a 2x2 wave grid; 128x128
    with 2x2, 4x1, 1x4 on 256 threads, 2x1, 1x2 on 128) for bf16, f16, fp8
    (e4m3) and int8 inputs, f32 / i32 output, in the four storage orders of A
    and B, at M = N = 8192, K = 4096;
  * attention forward (non-causal and causal, head_dim 64 and 128, bf16 and
    f16) at batch x heads x seq of the bench workloads.

The target of a row is the CU time one workgroup costs, in cycles:
y = t * f_sclk * CUs / workgroups (t the kernel's event-timed duration,
f_sclk the shader clock sampled while it runs).  The features of a row are
the solver's own, for the tile program one workgroup executes:

  * GEMM: the tile product C[bm, bn] += A[bm, bk] . B[bk, bn] with A and B
    staged from global memory into LDS, at the kernel's stage depth bk and
    the wave grid of the variant (the solver's contract for it must select
    that variant); the per-stage features are x(2 bk) - x(bk), the epilogue
    x(bk) - per-stage, and the row is K / bk stages plus one epilogue;
  * attention: the tensor-form tile program (Q.K^T, scale, row max, exp, row
    sum, divide, truncate, P.V, store) of the kernel's query block against
    one 64-key block and against two; the difference is one key block, and
    the row is the workgroup's key blocks plus the rest.

Per-wave features (MFMA, fragment reads, VALU, transcendental, cross-lane)
are scaled by waves / 4, the share of a CU's four SIMDs the workgroup
occupies, so the model is in CU cycles (the profile's `simd_share`).  The
fit is least squares on relative error with each weight bounded to a factor
BAND of its static hardware rate (unbounded, the attention rows' unmodelled
waits drive the cross-lane weight to thousands of cycles and the LDS weights
to zero); a feature that no row exercises keeps its default weight.  Beside
the fit the summary reports, per decision the solver makes on these tiles
(the wave grid of a 128x128 tile at fixed threads), the
grid each profile picks against the one that ran fastest.

Usage:
  python -m frisk_amd.calibrate measure --out SWEEP.json     (on the GPU)
  python -m frisk_amd.calibrate fit --sweep SWEEP.json --out PROFILE.json \\
      --summary SUMMARY.txt                                 (CPU)
"""
from __future__ import annotations

import argparse
import hashlib
import json
import sys
import time
from pathlib import Path
from typing import Dict, List, Optional, Tuple

from . import variants

PROFILE_DIR = Path(__file__).resolve().parent / "cost_profiles"
SWEEP_FILE = PROFILE_DIR / "cdna4-calibration-sweep.json"
PROFILE_FILE = PROFILE_DIR / "cdna4-calibrated-v1.json"

GEMM_SHAPE = (8192, 8192, 4096)
GEMM_DTYPES = ("bf16", "fp16", "fp8", "int8")
ORDERS = ((False, False), (False, True), (True, False), (True, True))
GEMM_VARIANTS = ((256, 2, 2), (128, 2, 2), (128, 4, 1), (128, 1, 4), (128, 2, 1), (128, 1, 2))
# (batch, heads, seq, head_dim, dtype, causal)
ATTN_CASES = ((4, 32, 4096, 128, "bf16", False), (4, 32, 4096, 64, "bf16", False),
              (4, 32, 4096, 128, "fp16", False), (8, 8, 2048, 64, "fp16", False),
              (4, 32, 4096, 128, "bf16", True), (4, 32, 4096, 64, "bf16", True))
ATTN_BN = 64  # keys per block of the attention kernel

# The tile-program element type of each input type (the session helper's
# names) and the accumulator / output type the sweep runs.
_TILE_DTYPE = {"bf16": "bf16", "fp16": "fp16", "fp8": "e4m3fn", "int8": "int8"}
_ACC = {"bf16": "fp32", "fp16": "fp32", "fp8": "fp32", "int8": "int32"}
_POLICY = {(2, 2): "Square", (4, 1): "FullRow", (1, 4): "FullCol", (2, 1): "FullRow",
           (1, 2): "FullCol"}


def _ir():
    from . import _ir as load
    return load()


# ---------------------------------------------------------------------------
# Solver features
# ---------------------------------------------------------------------------
def staged_tile_report(bm: int, bn: int, bk: int, dtype: str, trans_a: bool, trans_b: bool,
                       threads: int, policy: Optional[str], profile: Optional[str] = None) -> dict:
    """Layout inference's report for one workgroup's GEMM stage in tensor
    form: A and B copied from global memory into LDS, C[bm, bn] =
    op(A).op(B) on a frisk.mma, C stored.  `policy` names a GemmWarpPolicy
    (None: Auto, inference chooses the wave grid); `profile` is cost-profile
    JSON text (None: the default)."""
    import frisk_amd as F
    s = F.create_session()
    b = s.builder
    G, SH = F.MemorySpace.GLOBAL, F.MemorySpace.SHARED
    td, acc_t = _TILE_DTYPE[dtype], _ACC[dtype]
    ash = [bk, bm] if trans_a else [bm, bk]
    bsh = [bn, bk] if trans_b else [bk, bn]
    ga, gb = s.memref_type(ash, td, space=G), s.memref_type(bsh, td, space=G)
    gc = s.memref_type([bm, bn], acc_t, space=G)
    _, entry = s.new_kernel("stage", [ga, gb, gc])
    a, bb, c = (entry.get_argument(i) for i in range(3))
    i64 = b.get_int64_attr
    sa, sb = s.memref_type(ash, td, space=SH), s.memref_type(bsh, td, space=SH)
    par = b.create_parallel_op([1], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    alloc = lambda t: b.create_op("memref.alloc", [], [t], {"alignment": i64(1024)}).get_result(0)
    a_s, b_s = alloc(sa), alloc(sb)
    view = lambda x, t: b.create_op("frisk.layout_view", [x], [t]).get_result(0)
    empty = b.get_empty_affine_map()
    for src, dst, shape in ((view(a, ga), view(a_s, sa), ash), (view(bb, gb), view(b_s, sb), bsh)):
        b.create_copy_op(src, dst, [], [], empty, empty, shape, shape)
    acc_ty = b.get_ranked_tensor_ty(b.get_int32_ty() if acc_t == "int32" else b.get_f32_ty(), [bm, bn])
    zero = b.create_op("arith.constant", [], [acc_ty],
                       {"value": b.get_dense_splat_attr(acc_ty, 0 if acc_t == "int32" else 0.0)}
                       ).get_result(0)
    pol = b.get_gemm_warp_policy_attr(getattr(F.GemmWarpPolicy, policy or "Auto"))
    prod = b.create_op("frisk.mma", [view(a_s, sa), view(b_s, sb), zero], [acc_ty],
                       {"m": i64(bm), "n": i64(bn), "k": i64(bk),
                        "trans_a": b.get_bool_attr(trans_a), "trans_b": b.get_bool_attr(trans_b),
                        "policy": pol}).get_result(0)
    b.create_op("frisk.tile_store", [prod, view(c, gc)], [])
    s.module.set_attr("frisk.target", b.get_str_attr("gfx950"))
    if profile is None:
        return F.frisk.infer_layouts(s.module)
    return F.frisk.infer_layouts(s.module, cost_profile=profile)


def attention_tile_report(bm: int, bn: int, d: int, dtype: str, threads: int,
                          profile: Optional[str] = None) -> dict:
    """Layout inference's report for the tensor-form attention tile program
    of `bm` queries against `bn` keys (the structure of the reference's
    test/Transforms/attention-layout.mlir), waves along the queries."""
    import frisk_amd as F
    s = F.create_session()
    b = s.builder
    G, SH = F.MemorySpace.GLOBAL, F.MemorySpace.SHARED
    in_ty = {"fp16": b.get_f16_ty(), "bf16": b.get_bf16_ty()}[dtype]
    f32 = b.get_f32_ty()
    mq, mk = s.memref_type([bm, d], dtype, space=G), s.memref_type([bn, d], dtype, space=G)
    mo = s.memref_type([bm, d], "fp32", space=G)
    _, entry = s.new_kernel("attention", [mq, mk, mk, mo])
    q, k, v, o = (entry.get_argument(i) for i in range(4))
    i64 = b.get_int64_attr
    sq, sk = s.memref_type([bm, d], dtype, space=SH), s.memref_type([bn, d], dtype, space=SH)
    par = b.create_parallel_op([1], threads)
    b.set_insertion_point_to_start(par.add_entry_block())
    alloc = lambda t: b.create_op("memref.alloc", [], [t], {"alignment": i64(1024)}).get_result(0)
    qs, ks, vs = alloc(sq), alloc(sk), alloc(sk)
    view = lambda x, t: b.create_op("frisk.layout_view", [x], [t]).get_result(0)
    empty = b.get_empty_affine_map()
    for src, dst, rows in ((view(q, mq), view(qs, sq), bm), (view(k, mk), view(ks, sk), bn),
                           (view(v, mk), view(vs, sk), bn)):
        b.create_copy_op(src, dst, [], [], empty, empty, [rows, d], [rows, d])
    qv, kv, vv = view(qs, sq), view(ks, sk), view(vs, sk)
    t2 = lambda r, c, e: b.get_ranked_tensor_ty(e, [r, c])
    t1 = lambda r, e: b.get_ranked_tensor_ty(e, [r])
    const = lambda ty, x: b.create_op("arith.constant", [], [ty],
                                      {"value": b.get_dense_splat_attr(ty, x)}).get_result(0)
    op = lambda n, ins, ty, attrs=None: b.create_op(n, ins, [ty], attrs or {}).get_result(0)
    full_row = b.get_gemm_warp_policy_attr(F.GemmWarpPolicy.FullRow)
    sc = op("frisk.mma", [qv, kv, const(t2(bm, bn, f32), 0.0)], t2(bm, bn, f32),
            {"m": i64(bm), "n": i64(bn), "k": i64(d), "trans_a": b.get_bool_attr(False),
             "trans_b": b.get_bool_attr(True), "policy": full_row})
    sc = op("arith.mulf", [sc, const(t2(bm, bn, f32), 0.125)], t2(bm, bn, f32))
    mx = op("frisk.reduce_tensor", [sc], t1(bm, f32), {"kind": b.get_str_attr("max"), "dim": i64(1)})
    bmx = op("linalg.broadcast", [mx, op("tensor.empty", [], t2(bm, bn, f32))], t2(bm, bn, f32),
             {"dimensions": b.get_i64_array_attr([1])})
    ex = op("math.exp", [op("arith.subf", [sc, bmx], t2(bm, bn, f32))], t2(bm, bn, f32))
    sm = op("frisk.reduce_tensor", [ex], t1(bm, f32), {"kind": b.get_str_attr("sum"), "dim": i64(1)})
    bsm = op("linalg.broadcast", [sm, op("tensor.empty", [], t2(bm, bn, f32))], t2(bm, bn, f32),
             {"dimensions": b.get_i64_array_attr([1])})
    p = op("arith.truncf", [op("arith.divf", [ex, bsm], t2(bm, bn, f32))], t2(bm, bn, in_ty))
    out = op("frisk.mma", [p, vv, const(t2(bm, d, f32), 0.0)], t2(bm, d, f32),
             {"m": i64(bm), "n": i64(d), "k": i64(bn), "trans_a": b.get_bool_attr(False),
              "trans_b": b.get_bool_attr(False), "policy": full_row})
    b.create_op("frisk.tile_store", [out, view(o, mo)], [])
    s.module.set_attr("frisk.target", b.get_str_attr("gfx950"))
    if profile is None:
        return F.frisk.infer_layouts(s.module)
    return F.frisk.infer_layouts(s.module, cost_profile=profile)


def _sub(a: dict, b: dict, scale: float = 1.0) -> dict:
    keys = set(a) | set(b)
    return {k: a.get(k, 0.0) - scale * b.get(k, 0.0) for k in keys}


def _axpy(x: dict, n: float, y: dict) -> dict:
    keys = set(x) | set(y)
    return {k: x.get(k, 0.0) * n + y.get(k, 0.0) for k in keys}


def gemm_row_features(variant: Tuple[int, int, int], dtype: str, trans_a: bool, trans_b: bool,
                      bk: int, k: int) -> Tuple[dict, str]:
    """(features of one workgroup's whole K loop, the stage contract) for a
    GEMM kernel variant with stage depth bk over K = k."""
    tile, gm, gn = variant
    threads = 64 * gm * gn
    pol = _POLICY[(gm, gn)]
    r1 = staged_tile_report(tile, tile, bk, dtype, trans_a, trans_b, threads, pol)
    r2 = staged_tile_report(tile, tile, 2 * bk, dtype, trans_a, trans_b, threads, pol)
    contract = next(a for a in r1["assignments"] if a.startswith("mma#")).split(": ", 1)[1]
    got, why = variants.variant_for(contract, tile, tile, threads)
    if got != tuple(variant):
        raise ValueError(f"the solver's contract for variant {variant} selects {got}: {why}")
    step = _sub(r2["features"], r1["features"])
    epilogue = _sub(r1["features"], step)
    return _axpy(step, k // bk, epilogue), contract


def attention_row_features(d: int, dtype: str, waves: int, key_blocks: float) -> dict:
    """Features of one attention workgroup (32 queries per wave) that visits
    `key_blocks` blocks of 64 keys on average."""
    bm, threads = 32 * waves, 64 * waves
    r1 = attention_tile_report(bm, ATTN_BN, d, dtype, threads)
    r2 = attention_tile_report(bm, 2 * ATTN_BN, d, dtype, threads)
    block = _sub(r2["features"], r1["features"])
    rest = _sub(r1["features"], block)
    return _axpy(block, key_blocks, rest)


def attention_shape(b: int, h: int, s: int, causal: bool, d: int = 128,
                    cus: int = 256) -> Tuple[int, int, float]:
    """(waves per workgroup, workgroups, mean key blocks per workgroup) of
    the attention kernel's launch for a square (seq_q = seq_k = s) problem:
    head_dim 64 and below take 4 waves x 32 queries; head_dim 128 takes 8
    unless 4 finish sooner, counting workgroups of query blocks (under a
    causal mask, of pairs of them), the launch rule of
    frisk_amd/csrc/attn.h."""
    def workgroups(bm):
        q = -(-s // bm)
        return b * h * ((q + 1) // 2 if causal else q)
    w8, w4 = workgroups(256), workgroups(128)
    t8 = -(-w8 // cus)
    rest = w4 % (2 * cus)
    t4 = w4 // (2 * cus) + (0.0 if rest == 0 else 0.6 if rest <= cus else 1.0)
    waves = 4 if d <= 64 or t4 < t8 else 8
    bm = 32 * waves
    qb = -(-s // bm)
    if causal:
        # Query block i sees keys [0, (i + 1) bm): (i + 1) bm / 64 blocks.
        blocks = sum(min(-(-(i + 1) * bm // ATTN_BN), -(-s // ATTN_BN)) for i in range(qb)) / qb
    else:
        blocks = -(-s // ATTN_BN)
    return waves, b * h * qb, float(blocks)


def row_features(row: dict) -> dict:
    """The solver's features of one workgroup of a sweep row."""
    if row["kind"] == "gemm":
        return gemm_row_features(tuple(row["variant"]), row["dtype"], row["trans_a"],
                                 row["trans_b"], row["bk"], row["k"])[0]
    return attention_row_features(row["d"], row["dtype"], row["waves"], row["key_blocks"])


def row_waves(row: dict) -> int:
    if row["kind"] == "gemm":
        return row["variant"][1] * row["variant"][2]
    return row["waves"]


# ---------------------------------------------------------------------------
# Measurement (GPU)
# ---------------------------------------------------------------------------
def _time_launches(torch, fn, window_ms: float = 200.0) -> Tuple[float, Optional[int]]:
    """(event-timed mean duration in ms, median shader clock in MHz) of
    back-to-back launches of fn over about `window_ms`, after about 150 ms
    of the same launches to let the clock settle.  The clock is sampled
    every 10 ms during the timed launches."""
    import threading
    from .clock import read_sclk_mhz
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    once = max(time.perf_counter() - t0, 3e-6) / 3 * 1e3
    for _ in range(max(1, int(150.0 / once))):
        fn()
    reps = max(5, min(4000, int(window_ms / once)))
    samples, stop = [], threading.Event()

    def sample():
        while not stop.is_set():
            v = read_sclk_mhz()
            if v is not None:
                samples.append(v)
            time.sleep(0.01)

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    th = threading.Thread(target=sample, daemon=True)
    th.start()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    stop.set()
    th.join()
    samples.sort()
    return a.elapsed_time(b) / reps, (samples[len(samples) // 2] if samples else None)


def _summarize(got):
    """(mean ms, mean MHz, relative spread of the cycle counts) of timed
    windows [(ms, MHz), ...] of one launch."""
    ms = sum(g[0] for g in got) / len(got)
    clocks = [g[1] for g in got if g[1] is not None]
    mhz = round(sum(clocks) / len(clocks)) if clocks else None
    cyc = [g[0] * (g[1] or 1) for g in got]
    return ms, mhz, round((max(cyc) - min(cyc)) / (sum(cyc) / len(got)), 4)


def _timed_passes(torch, fn, passes: int = 2):
    """_summarize of `passes` timed windows of fn."""
    return _summarize([_time_launches(torch, fn) for _ in range(passes)])


def _timed_interleaved(torch, fns, passes: int = 3):
    """_summarize per launch of `passes` rounds that time every fn once in
    turn, so that a drift of the clock between rounds reaches all of them
    alike (the wave grids of one group differ by a few percent)."""
    got = [[] for _ in fns]
    for _ in range(passes):
        for i, fn in enumerate(fns):
            got[i].append(_time_launches(torch, fn))
    return [_summarize(g) for g in got]


def measure(out: Path) -> dict:
    import torch
    from . import runtime as rt
    from .build import source_digest
    rt.load()
    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)
    cus = props.multi_processor_count
    fp8 = torch.float8_e4m3fn
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp8": fp8, "int8": torch.int8}
    odt = {"bf16": torch.float32, "fp16": torch.float32, "fp8": torch.float32, "int8": torch.int32}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2026)
    rows: List[dict] = []
    m, n, k = GEMM_SHAPE
    for dt in GEMM_DTYPES:
        if dt == "int8":
            mk = lambda *sh: torch.randint(-8, 8, sh, generator=gen, device="cuda", dtype=torch.int8)
        else:
            mk = lambda *sh: (torch.randn(*sh, generator=gen, device="cuda") * 0.5).to(tdt[dt])
        for ta, tb in ORDERS:
            a = mk(k, m) if ta else mk(m, k)
            b = mk(n, k) if tb else mk(k, n)
            c = torch.empty(m, n, device="cuda", dtype=odt[dt])
            fns = [lambda var=var: rt.gemm(a, b, c, trans_a=ta, trans_b=tb, workspace=False,
                                           variant=var) for var in GEMM_VARIANTS]
            if not rows:
                _time_launches(torch, fns[0], window_ms=1000.0)  # the clock's first ramp
            timed = _timed_interleaved(torch, fns)
            for var, (ms, mhz, spread) in zip(GEMM_VARIANTS, timed):
                plan = rt.gemm_plan(a, b, c, trans_a=ta, trans_b=tb, workspace=False, variant=var)
                ct = variants.parse_contract(plan["mma_contract"])
                atom_k = int(ct["atom"].rsplit("x", 1)[1].split("_")[0])
                bk = ct["repeats"][2] * atom_k
                wgs = -(-m // var[0]) * -(-n // var[0])
                rows.append({"kind": "gemm", "dtype": dt, "trans_a": ta, "trans_b": tb,
                             "variant": list(var), "m": m, "n": n, "k": k, "bk": bk,
                             "kernel": plan["kernel"], "workgroups": wgs, "ms": round(ms, 6),
                             "sclk_mhz": mhz, "pass_spread": spread})
                print(f"gemm {dt} ta={int(ta)} tb={int(tb)} {var}: {ms * 1e3:.1f} us "
                      f"at {mhz} MHz", flush=True)
            del a, b, c
    for (bb, h, s, d, dt, causal) in ATTN_CASES:
        q, kk, v = (torch.randn(bb, h, s, d, generator=gen, device="cuda").to(tdt[dt]) for _ in range(3))
        o = torch.empty_like(q)
        fn = lambda: rt.attn_fwd(q, kk, v, o, causal=causal)
        waves, wgs, blocks = attention_shape(bb, h, s, causal, d, cus)
        ms, mhz, spread = _timed_passes(torch, fn)
        rows.append({"kind": "attention", "dtype": dt, "batch": bb, "heads": h, "seq": s, "d": d,
                     "causal": causal, "waves": waves, "workgroups": wgs, "key_blocks": blocks,
                     "ms": round(ms, 6), "sclk_mhz": mhz, "pass_spread": spread})
        print(f"attention b{bb} h{h} s{s} d{d} {dt} causal={causal}: {ms * 1e3:.1f} us "
              f"at {mhz} MHz", flush=True)
        del q, kk, v, o
    sweep = {"gpu": {"name": props.name, "arch": getattr(props, "gcnArchName", None), "cus": cus},
             "source_sha256_16": source_digest(), "torch": torch.__version__,
             "hip": torch.version.hip, "rows": rows}
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(sweep, indent=1) + "\n")
    return sweep


# ---------------------------------------------------------------------------
# Fit (CPU)
# ---------------------------------------------------------------------------
def target_cycles(row: dict, cus: int) -> float:
    """CU cycles per workgroup: kernel time x shader clock x CUs / workgroups."""
    return row["ms"] * 1e-3 * row["sclk_mhz"] * 1e6 * cus / row["workgroups"]


def design_matrix(rows: List[dict], simd_share: bool):
    """Feature matrix (rows x features) as the solver weighs it: per-wave
    features scaled by waves / 4 when simd_share."""
    import numpy as np
    defaults = _ir().frisk.cost_profile_defaults()
    names, per_wave = list(defaults["weights"]), set(defaults["per_wave"])
    x = np.zeros((len(rows), len(names)))
    for i, r in enumerate(rows):
        share = row_waves(r) / 4.0 if simd_share else 1.0
        for j, f in enumerate(names):
            x[i, j] = r["features"].get(f, 0.0) * (share if f in per_wave else 1.0)
    return x, names


BAND = 4.0  # each fitted weight stays within [w0 / BAND, w0 * BAND] of its static rate w0


def _fit_relative(x, y, w0):
    """Least squares on relative error, each weight bounded to the band
    around its static (hardware-rate) weight w0."""
    import numpy as np
    from scipy.optimize import lsq_linear
    a = x / y[:, None]
    w0 = np.asarray(w0, dtype=float)
    return lsq_linear(a, np.ones(len(y)), bounds=(w0 / BAND, w0 * BAND), method="bvls").x


def canonical_weights(weights: Dict[str, float]) -> str:
    return json.dumps({k: weights[k] for k in sorted(weights)}, sort_keys=True,
                      separators=(",", ":"))


def profile_text(profile: dict) -> str:
    """The cost-profile JSON that frisk.infer_layouts reads."""
    return json.dumps(profile, indent=1, sort_keys=True) + "\n"


NEAR = 0.02  # grids within 2% of the fastest count as fast as it (timing spread)


def decisions(rows: List[dict], profiles: Dict[str, Optional[str]]) -> List[dict]:
    """For each group of 128x128 GEMM rows that differ only in the wave grid
    at fixed threads: the fastest measured grid, those within NEAR of it,
    and the grid layout inference picks (Auto policy) under each profile."""
    groups: Dict[tuple, List[dict]] = {}
    for r in rows:
        if r["kind"] == "gemm" and r["variant"][0] == 128:
            key = (r["dtype"], r["trans_a"], r["trans_b"], r["variant"][1] * r["variant"][2])
            groups.setdefault(key, []).append(r)
    out = []
    for (dt, ta, tb, waves), g in sorted(groups.items()):
        best = min(g, key=lambda r: r["ms"])
        grid = lambda r: f"{r['variant'][1]}x{r['variant'][2]}"
        rec = {"dtype": dt, "trans_a": ta, "trans_b": tb, "threads": 64 * waves,
               "measured": {grid(r): r["ms"] for r in g}, "fastest": grid(best),
               "near": sorted(grid(r) for r in g if r["ms"] <= best["ms"] * (1 + NEAR)),
               "picked": {}}
        for name, text in profiles.items():
            rep = staged_tile_report(128, 128, best["bk"], dt, ta, tb, 64 * waves, None, text)
            contract = next(a for a in rep["assignments"] if a.startswith("mma#")).split(": ", 1)[1]
            lm, ln = variants.logical_grid(variants.parse_contract(contract))
            rec["picked"][name] = f"{lm}x{ln}"
        out.append(rec)
    return out


def fit(sweep: dict, *, with_decisions: bool = True) -> Tuple[dict, dict]:
    """(profile, report) fitted to the sweep's rows."""
    import numpy as np
    cus = int(sweep["gpu"]["cus"])
    rows = sweep["rows"]
    for r in rows:
        r["features"] = {k: v for k, v in row_features(r).items() if v}
    y = np.array([target_cycles(r, cus) for r in rows])
    x, names = design_matrix(rows, simd_share=True)
    excited = [j for j in range(len(names)) if np.any(x[:, j] != 0)]
    defaults = _ir().frisk.cost_profile_defaults()["weights"]
    w0 = [defaults[names[j]] for j in excited]
    w_exc = _fit_relative(x[:, excited], y, w0)
    weights = dict(defaults)
    for j, wj in zip(excited, w_exc):
        weights[names[j]] = float(f"{wj:.6g}")
    wv = np.array([weights[f] for f in names])
    pred = x @ wv
    rel = pred / y - 1
    # Leave-one-out relative error of the same fit.
    loo = []
    for i in range(len(rows)):
        keep = np.arange(len(rows)) != i
        wi = _fit_relative(x[keep][:, excited], y[keep], w0)
        loo.append(float(x[i, excited] @ wi / y[i] - 1))
    loo = np.array(loo)
    x0, _ = design_matrix(rows, simd_share=False)
    pred0 = x0 @ np.array([defaults[f] for f in names])
    # The default profile's scale is arbitrary: compare its shape after the
    # best single scale factor (least squares on relative error).
    s0 = float(np.sum(pred0 / y) / np.sum((pred0 / y) ** 2))
    rel0 = s0 * pred0 / y - 1
    digest = hashlib.sha256(canonical_weights(weights).encode()).hexdigest()
    profile = {
        "id": f"cdna4-calibrated-v1-{digest[:16]}",
        "simd_share": True,
        "weights": weights,
        "provenance": {
            "sweep": SWEEP_FILE.name,
            "sweep_rows": len(rows),
            "gpu": sweep["gpu"],
            "source_sha256_16": sweep.get("source_sha256_16"),
            "target": "CU cycles per workgroup = t * f_sclk * CUs / workgroups",
            "fit": "least squares on relative error, each weight within a factor "
                   f"{BAND:g} of its cdna4-layout-v1 rate; unexercised features keep that weight",
            "fitted_features": [names[j] for j in excited],
            "rel_rms": round(float(np.sqrt(np.mean(rel ** 2))), 4),
            "loo_rel_rms": round(float(np.sqrt(np.mean(loo ** 2))), 4),
            "weights_sha256": digest,
        },
    }
    report = {"rows": rows, "y": y.tolist(), "pred": pred.tolist(), "rel": rel.tolist(),
              "loo": loo.tolist(), "default_scale": s0, "default_rel": rel0.tolist(),
              "names": names, "excited": [names[j] for j in excited], "weights": weights,
              "defaults": defaults}
    if with_decisions:
        report["decisions"] = decisions(rows, {"cdna4-layout-v1": None,
                                               profile["id"]: profile_text(profile)})
    return profile, report


def summary_text(profile: dict, report: dict, command: str) -> str:
    import numpy as np
    lines = [f"# Cost-model calibration: {profile['id']}", "",
             "Sweep: python -m frisk_amd.calibrate measure --out "
             "frisk_amd/cost_profiles/cdna4-calibration-sweep.json (on the MI355X)",
             f"Fit: {command}", "",
             f"GPU: {profile['provenance']['gpu']}; rows: {len(report['rows'])}; target: "
             f"{profile['provenance']['target']}.", "",
             "## Weights (cycles per unit; per-wave features scaled by waves / 4)", "",
             f"{'feature':22s} {'cdna4-layout-v1':>16s} {'calibrated':>12s}"]
    for f in report["names"]:
        tag = "" if f in report["excited"] else "   (not exercised: default kept)"
        lines.append(f"{f:22s} {report['defaults'][f]:16.6g} {report['weights'][f]:12.6g}{tag}")
    rel, loo, rel0 = (np.array(report[k]) for k in ("rel", "loo", "default_rel"))
    rms = lambda v: float(np.sqrt(np.mean(v ** 2)))
    lines += ["", "## Fit", "",
              f"relative error, calibrated: rms {rms(rel):.3f}, max |.| {np.max(np.abs(rel)):.3f}; "
              f"leave-one-out rms {rms(loo):.3f}",
              f"relative error, cdna4-layout-v1 (best scale {report['default_scale']:.3g}): "
              f"rms {rms(rel0):.3f}, max |.| {np.max(np.abs(rel0)):.3f}", "",
              f"{'row':44s} {'ms':>9s} {'y cycles':>10s} {'calib':>7s} {'v1':>7s}"]
    for r, y, e, e0 in zip(report["rows"], report["y"], rel, rel0):
        if r["kind"] == "gemm":
            name = (f"gemm {r['dtype']} {'t' if r['trans_a'] else 'n'}{'t' if r['trans_b'] else 'n'} "
                    f"{r['variant'][0]} {r['variant'][1]}x{r['variant'][2]}")
        else:
            name = (f"attn b{r['batch']}h{r['heads']}s{r['seq']}d{r['d']} {r['dtype']}"
                    f"{' causal' if r['causal'] else ''} w{r['waves']}")
        lines.append(f"{name:44s} {r['ms']:9.4f} {y:10.0f} {e:+7.3f} {e0:+7.3f}")
    if "decisions" in report:
        lines += ["", "## Wave-grid decisions (128x128 tile, Auto policy)", "",
                  f"{'group':24s} {'fastest':>8s} " + " ".join(f"{k[:24]:>26s}" for k in
                                                          report["decisions"][0]["picked"])]
        agree = {k: 0 for k in report["decisions"][0]["picked"]}
        near = dict(agree)
        for d in report["decisions"]:
            g = f"{d['dtype']} {'t' if d['trans_a'] else 'n'}{'t' if d['trans_b'] else 'n'} {d['threads']}thr"
            lines.append(f"{g:24s} {d['fastest']:>8s} " +
                         " ".join(f"{v:>26s}" for v in d["picked"].values()) +
                         f"   within {NEAR:.0%}: {','.join(d['near'])}")
            for k, v in d["picked"].items():
                agree[k] += v == d["fastest"]
                near[k] += v in d["near"]
        lines.append("")
        for k in agree:
            lines.append(f"{k}: picks the fastest grid in {agree[k]} of {len(report['decisions'])} "
                         f"groups, one within {NEAR:.0%} of it in {near[k]}")
    return "\n".join(lines) + "\n"


def load_profile(name_or_path: str) -> str:
    """Cost-profile JSON text: a file path, or the name of a profile shipped
    in frisk_amd/cost_profiles (with or without .json; a calibrated
    profile's id also names its file's profile)."""
    p = Path(name_or_path)
    if p.is_file():
        return p.read_text()
    for cand in sorted(PROFILE_DIR.glob("*.json")):
        if cand.name == SWEEP_FILE.name:
            continue
        if name_or_path in (cand.stem, cand.name):
            return cand.read_text()
        try:
            if json.loads(cand.read_text()).get("id") == name_or_path:
                return cand.read_text()
        except ValueError:
            continue
    raise FileNotFoundError(f"cost profile {name_or_path!r}: no such file or shipped profile")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m frisk_amd.calibrate")
    sub = ap.add_subparsers(dest="cmd", required=True)
    m = sub.add_parser("measure", help="time the sweep's kernels on the GPU")
    m.add_argument("--out", type=Path, default=SWEEP_FILE)
    f = sub.add_parser("fit", help="fit a cost profile to a measured sweep")
    f.add_argument("--sweep", type=Path, default=SWEEP_FILE)
    f.add_argument("--out", type=Path, default=PROFILE_FILE)
    f.add_argument("--summary", type=Path, default=None)
    args = ap.parse_args(argv)
    if args.cmd == "measure":
        measure(args.out)
        return 0
    sweep = json.loads(args.sweep.read_text())
    profile, report = fit(sweep)
    args.out.write_text(profile_text(profile))
    if args.summary:
        cmd = "python -m frisk_amd.calibrate fit " + " ".join(
            a if " " not in a else repr(a) for a in (argv if argv is not None else sys.argv[1:])[1:])
        args.summary.write_text(summary_text(profile, report, cmd))
    print(json.dumps(profile["provenance"], indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
