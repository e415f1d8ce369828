"""Run a frisk tile program on the GPU through the C-ABI.

The reference has no in-process execution (ffi/ffi.cpp:6 leaves it out; its
programs run out of process through an exported packet).  Here
`execute(module, kernel, tensors)` recognises the two tile programs of the
GEMM / attention path, proves from the IR that the program computes the
whole-tensor operation, and launches the MI355X kernel for it:

* GEMM (`frisk_gemm`), in two forms:
  - whole-matrix: the kernel body is `frisk.gemm(A, B, C)` on kernel
    arguments, optionally preceded by `frisk.fill(C, 0)`;
  - tiled (the tile program of the reference's tmp/ir.mlir:2-16): one
    2-D `frisk.parallel` over (M/BM, N/BN) tiles holding a zero-filled Local
    accumulator, a `frisk.for` over K/BK whose body copies the A and B tiles
    into Shared buffers and accumulates `frisk.gemm` into the accumulator,
    and a final copy of the accumulator into C.  The copy index maps must be
    affine in the loop indices and place the tiles so that the grid covers
    C exactly once and the loop covers K exactly once (checked below).
* Attention (`frisk_attn_fwd`): the online-softmax skeleton of
  tmp/ir.mlir:89-157 expressed with the builder's ops: a 3-D
  `frisk.parallel` over (B, H, S/BM) that copies the Q tile, fills the
  output accumulator (0), the row maxima (-inf) and row sums (0), loops over
  key blocks copying the K tile, forming scores with `frisk.gemm(q, k, s)`,
  reducing them into the row maxima (max) and sums (add), casting them to
  the input dtype, copying the V tile and accumulating `frisk.gemm(p, v,
  o)`, and finally copies the accumulator into O.  The rescaling steps the
  builder cannot express (exp2 of scaled scores, accumulator rescale and the
  final division) are implied by that skeleton; `frisk.block` ops standing
  for them are allowed in the loop.  `sm_scale` (default 1/sqrt(D)) and
  `causal` are arguments of execute().

The kernel that runs comes from layout decisions made here, not inside the
library:

* A tiled GEMM program names its workgroup tile (BM x BN) and thread count.
  `plan()` runs layout inference (frisk_amd/ir/infer.cpp) on a copy of the
  program and reads the instruction contract of its tile product (MFMA atom
  and wave grid, `#frisk.mma_contract`); when a compiled kernel executes
  exactly that workgroup product (frisk_amd/variants.py) `execute()` runs
  that variant (`frisk_gemm_desc.tile / wave_m / wave_n`, and the K slices
  the launch contract gives the same tile and grid).
* A whole-matrix GEMM takes the gfx950 target's launch contract
  (`F.frisk.gemm_launch_plan`: kernel, workgroup tile, wave grid, stage
  depth, K slices; launch_plan.h, shared with the C-ABI), then the
  instruction contract inference solves for that workgroup tile under the
  op's warp policy, and `execute()` requests that variant with those slices.
  The small-M and generic kernels have no tile program: their launch
  contract names them and the library runs them.
* Attention takes the waves per workgroup from the target's attention
  launch contract (`F.frisk.attention_launch_plan`) and requests them.

Every request is checked against the C-ABI first (`frisk_gemm_plan`): when
the tensors do not meet a variant's conditions (alignment, pitches) the
library's own choice runs and `mismatch` says why; `layouts_match` is False
whenever the kernel that runs is not the one the contracts name.  Packets
(`execute_packet`) follow the same rule.  Anything else raises ValueError
naming the first mismatch.  There is no CPU fallback.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from functools import lru_cache
from typing import Optional, Sequence

from . import _ir, tileprog, variants

ir = _ir()
fr = ir.frisk


@dataclass
class GemmPlan:
    a: int
    b: int
    c: int
    trans_a: bool
    trans_b: bool
    clear_accum: bool
    m: int
    n: int
    k: int
    # The tile product's instruction contract from layout inference, the
    # kernel variant (tile, wave_m, wave_n) that executes it, or why none does.
    contract: Optional[str] = None
    variant: Optional[tuple] = None
    layouts_match: bool = False
    mismatch: str = ""
    # The program's workgroup tile (bm, bn, bk, dtype, policy, threads), or
    # None for a whole-matrix program.
    tile: Optional[tuple] = field(default=None, repr=False)
    # The launch contract of the GEMM (the target's gemm_launch_plan); the
    # variant above carries its K slices when it runs that tile and grid.
    launch: Optional[dict] = None
    # Whether the MFMA kernel's LDS swizzle of each K-major operand is the
    # layout target's proposal for its stage rows (None: nothing to check).
    swizzle_match: Optional[bool] = None
    # A / B and C element types (IR spelling), and the GEMM's warp policy.
    elems: Optional[tuple] = field(default=None, repr=False)
    policy: object = field(default=None, repr=False)


@dataclass
class AttnPlan:
    q: int
    k: int
    v: int
    o: int
    k_transposed: bool
    batch: int
    heads: int
    seq: int
    head_dim: int
    # Waves per workgroup from the attention launch contract (causal and
    # non-causal: causal is an argument of execute()).
    waves: Optional[dict] = None


class _Reject(ValueError):
    pass


def _fail(msg: str):
    raise _Reject(msg)


def _body_ops(block) -> list:
    return [op for op in block.get_operations() if op.get_name() != "frisk.end"]


def _arg_index(value, entry) -> Optional[int]:
    owner = getattr(value, "get_owner", None)
    if owner is None:
        return None
    if value.get_owner().id() != entry.id():
        return None
    return value.get_arg_number()


def _shape(value):
    return list(value.get_type().get_shape())


def _elem(value):
    return str(value.get_type().get_element_ty())


def _space(value):
    return value.get_type().get_memory_space()


# ---------------------------------------------------------------------------
# Affine index analysis
# ---------------------------------------------------------------------------
class _Ivs:
    """Loop indices in scope: parallel ivs range over [0, grid), the for iv
    over lower, lower + step, ... < upper."""

    def __init__(self):
        self.ranges = {}  # (block id, arg number) -> list of values (first, next, last)

    def add_parallel(self, par):
        block = par.get_region(0).front()
        for i, extent in enumerate(par.get_grid()):
            self.ranges[(block.id(), i)] = (0, 1, extent)
        return block

    def add_for(self, loop):
        block = loop.get_region(0).front()
        lo, hi, st = loop.get_lower_bound(), loop.get_upper_bound(), loop.get_step()
        if st <= 0 or hi <= lo:
            _fail(f"frisk.for {lo} to {hi} step {st} is empty or has a non-positive step")
        self.ranges[(block.id(), 0)] = (lo, st, (hi - lo + st - 1) // st)
        return block

    def key(self, value):
        if not hasattr(value, "get_owner"):
            _fail("copy indices must be loop induction variables")
        k = (value.get_owner().id(), value.get_arg_number())
        if k not in self.ranges:
            _fail("copy index is not a parallel or for induction variable in scope")
        return k


def _origin(ivs: _Ivs, amap, indices, rank: int) -> tuple[list[int], dict]:
    """Affine form of a copy's tile origin: (constant vector, {iv: coefficient
    vector per trip}), coefficients per trip of the loop (step applied).  An
    empty map (whole-buffer copy) is the origin 0."""
    if amap.get_num_results() == 0:
        return [0] * rank, {}
    if amap.get_num_results() != rank:
        _fail(f"copy map {amap} must give one offset per dimension ({rank})")
    if amap.get_num_symbols():
        _fail("copy maps with symbols are not supported")
    for e in amap.get_results():
        if not e.is_pure_affine():
            _fail(f"copy map result {e} is not pure affine")
    keys = [ivs.key(v) for v in indices]
    base = [ivs.ranges[k][0] for k in keys]
    c0 = amap.evaluate(base)
    coef = {}
    for k in set(keys):
        step = ivs.ranges[k][1]
        pt = [b + (step if keys[i] == k else 0) for i, b in enumerate(base)]
        d = [x - y for x, y in zip(amap.evaluate(pt), c0)]
        if any(d):
            coef[k] = d
    return c0, coef


def _tile_copy(op, ivs: _Ivs):
    """(src, dst, src origin affine form, dst origin affine form, extents) of a copy."""
    cp = fr.CopyOp.from_operation(op)
    src, dst = cp.get_src_memref(), cp.get_dst_memref()
    so = _origin(ivs, cp.get_src_affine_map(), list(cp.get_src_indices()), len(_shape(src)))
    do = _origin(ivs, cp.get_dst_affine_map(), list(cp.get_dst_indices()), len(_shape(dst)))
    return src, dst, so, do, list(cp.get_src_extents()), list(cp.get_dst_extents())


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def _gemm_whole(ops, entry) -> GemmPlan:
    fill_c = None
    if len(ops) == 2 and ops[0].get_name() == "frisk.fill":
        fill_c = ops[0]
        ops = ops[1:]
    if len(ops) != 1 or ops[0].get_name() != "frisk.gemm":
        _fail("not a whole-matrix GEMM")
    g = fr.GemmOp.from_operation(ops[0])
    idx = [_arg_index(v, entry) for v in (g.get_matrix_A(), g.get_matrix_B(), g.get_matrix_C())]
    if None in idx:
        _fail("whole-matrix GEMM operands must be kernel arguments")
    op = ops[0]
    clear = bool(op.get_attr("clear_accum"))
    if fill_c is not None:
        if fill_c.get_operand(0) != g.get_matrix_C() or fill_c.get_attr("value") != 0.0:
            _fail("only a zero fill of C may precede the GEMM")
        clear = True
    return GemmPlan(idx[0], idx[1], idx[2], bool(op.get_attr("transA")), bool(op.get_attr("transB")),
                    clear, op.get_attr("M"), op.get_attr("N"), op.get_attr("K"),
                    elems=(_elem(g.get_matrix_A()), _elem(g.get_matrix_C())),
                    policy=op.get_attr("policy"))


def _gemm_tiled(ops, entry) -> GemmPlan:
    if len(ops) != 1 or ops[0].get_name() != "frisk.parallel":
        _fail("not a tiled GEMM (expected one frisk.parallel)")
    par = fr.ParallelOp.from_operation(ops[0])
    grid = par.get_grid()
    if len(grid) != 2:
        _fail("tiled GEMM needs a 2-D parallel grid")
    ivs = _Ivs()
    pblock = ivs.add_parallel(par)
    body = _body_ops(pblock)
    allocs = {}
    i = 0
    while i < len(body) and body[i].get_name() == "frisk.alloc_buffer":
        allocs[body[i].get_result(0).id()] = body[i].get_result(0)
        i += 1
    rest = body[i:]
    names = [o.get_name() for o in rest]
    if names != ["frisk.fill", "frisk.for", "frisk.copy"]:
        _fail(f"tiled GEMM body must be allocs, fill, for, copy (found {names})")
    fill, loop_op, store = rest
    acc = fill.get_operand(0)
    if acc.id() not in allocs or _space(acc) != ir.MemorySpace.LOCAL or fill.get_attr("value") != 0.0:
        _fail("the accumulator must be a zero-filled Local buffer")
    loop = fr.ForOp.from_operation(loop_op)
    lblock = ivs.add_for(loop)
    lops = _body_ops(lblock)
    if sorted(o.get_name() for o in lops) != ["frisk.copy", "frisk.copy", "frisk.gemm"] or \
            lops[-1].get_name() != "frisk.gemm":
        _fail("the K loop must copy the A and B tiles, then accumulate one frisk.gemm")
    gop = lops[-1]
    g = fr.GemmOp.from_operation(gop)
    a_t, b_t, c_t = g.get_matrix_A(), g.get_matrix_B(), g.get_matrix_C()
    if c_t != acc or gop.get_attr("clear_accum"):
        _fail("the loop GEMM must accumulate (clear_accum = false) into the filled accumulator")
    ta, tb = bool(gop.get_attr("transA")), bool(gop.get_attr("transB"))
    bm, bn, bk = gop.get_attr("M"), gop.get_attr("N"), gop.get_attr("K")
    loads = {}
    for cop in lops[:2]:
        src, dst, so, do, sext, dext = _tile_copy(cop, ivs)
        if dst.id() not in allocs or do[1] or any(do[0]):
            _fail("tile loads must fill a whole Shared/Local tile buffer")
        loads[dst.id()] = (src, so, sext)
    if a_t.id() not in loads or b_t.id() not in loads:
        _fail("the GEMM operands must be the tiles loaded in the loop")
    a_src, a_org, a_ext = loads[a_t.id()]
    b_src, b_org, b_ext = loads[b_t.id()]
    ia, ib = _arg_index(a_src, entry), _arg_index(b_src, entry)
    if ia is None or ib is None:
        _fail("tiles must be loaded from kernel arguments")
    src, dst, so, do, sext, dext = _tile_copy(store, ivs)
    ic = _arg_index(dst, entry)
    if src != acc or ic is None or so[1] or any(so[0]):
        _fail("the accumulator must be stored into a kernel argument")
    if sext != [bm, bn] or dext != [bm, bn]:
        _fail(f"the C store must copy a {bm}x{bn} tile (extents {sext} / {dext})")

    kkey = (lblock.id(), 0)
    trips = ivs.ranges[kkey][2]
    pkeys = [(pblock.id(), 0), (pblock.id(), 1)]
    # Positions of (M, K) in A's storage and (K, N) in B's.
    am, ak = (1, 0) if ta else (0, 1)
    bk_, bn_ = (1, 0) if tb else (0, 1)

    def per_trip(org, dim, key):
        return org[1].get(key, [0, 0])[dim]

    a0, b0, c0 = a_org[0], b_org[0], do[0]
    # K tiles: A and B advance by BK per trip from 0, and nothing else moves K.
    for name, org, kd in (("A", a_org, ak), ("B", b_org, bk_)):
        if org[0][kd] != 0 or per_trip(org, kd, kkey) != bk:
            _fail(f"{name} tile K offset must start at 0 and advance by {bk} per trip")
        if any(per_trip(org, kd, p) for p in pkeys):
            _fail(f"{name} tile K offset must not depend on the grid")
    # M and N tiles: one grid axis each, stride BM / BN, never the K loop.
    m_axes = [p for p in pkeys if per_trip(a_org, am, p)]
    n_axes = [p for p in pkeys if per_trip(b_org, bn_, p)]
    if len(m_axes) != 1 or len(n_axes) != 1 or m_axes == n_axes:
        _fail("A's M offset and B's N offset must each follow a different grid axis")
    pm, pn = m_axes[0], n_axes[0]
    if a0[am] != 0 or per_trip(a_org, am, pm) != bm or per_trip(a_org, am, kkey):
        _fail(f"A tile M offset must be {bm} * grid index")
    if b0[bn_] != 0 or per_trip(b_org, bn_, pn) != bn or per_trip(b_org, bn_, kkey):
        _fail(f"B tile N offset must be {bn} * grid index")
    if c0 != [0, 0] or per_trip(do, 0, pm) != bm or per_trip(do, 1, pn) != bn or \
            per_trip(do, 0, pn) or per_trip(do, 1, pm) or kkey in do[1]:
        _fail("C tile origin must be (BM * m-index, BN * n-index)")
    a_shape, b_shape, c_shape = _shape(a_src), _shape(b_src), _shape(dst)
    M, K = (a_shape[1], a_shape[0]) if ta else (a_shape[0], a_shape[1])
    N = b_shape[0] if tb else b_shape[1]
    gm, gn = grid[pm[1]], grid[pn[1]]
    if gm * bm != M or gn * bn != N or trips * bk != K or c_shape != [M, N]:
        _fail(f"grid {grid} x tile {bm}x{bn}x{bk} x {trips} trips does not cover "
              f"A{a_shape} B{b_shape} C{c_shape} exactly")
    if _elem(a_t) != _elem(a_src) or _elem(b_t) != _elem(b_src):
        _fail("A/B tiles must keep the input dtype")
    tile = (bm, bn, bk, _HELPER_NAMES.get(_elem(a_t), _elem(a_t)), gop.get_attr("policy"),
            par.get_thread_num())
    return GemmPlan(ia, ib, ic, ta, tb, True, M, N, K, tile=tile,
                    elems=(_elem(a_src), _elem(dst)), policy=gop.get_attr("policy"))


# Element type (IR spelling) -> the session helper's dtype name.
_HELPER_NAMES = {"f16": "fp16", "bf16": "bf16", "f8E4M3FN": "e4m3fn", "i8": "int8", "f32": "fp32"}
_ESIZE = {"fp16": 2, "bf16": 2, "e4m3fn": 1, "int8": 1, "fp32": 4}


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def _attention(ops, entry) -> AttnPlan:
    if len(ops) != 1 or ops[0].get_name() != "frisk.parallel":
        _fail("not an attention program (expected one frisk.parallel)")
    par = fr.ParallelOp.from_operation(ops[0])
    grid = par.get_grid()
    if len(grid) != 3:
        _fail("attention needs a 3-D (batch, heads, query blocks) grid")
    ivs = _Ivs()
    pblock = ivs.add_parallel(par)
    pk = [(pblock.id(), i) for i in range(3)]
    body = _body_ops(pblock)
    allocs = {o.get_result(0).id(): o.get_result(0) for o in body if o.get_name() == "frisk.alloc_buffer"}
    rest = [o for o in body if o.get_name() not in ("frisk.alloc_buffer", "arith.constant")]
    loops = [o for o in rest if o.get_name() == "frisk.for"]
    if len(loops) != 1:
        _fail("attention needs exactly one key-block loop")
    li = rest.index(loops[0])
    pre, post = rest[:li], rest[li + 1:]
    loop = fr.ForOp.from_operation(loops[0])
    lblock = ivs.add_for(loop)
    kkey = (lblock.id(), 0)
    lops = [o for o in _body_ops(lblock) if o.get_name() != "frisk.block"]

    # Prologue: the Q tile load and the accumulator / statistics fills.
    q_load = [o for o in pre if o.get_name() == "frisk.copy"]
    fills = {o.get_operand(0).id(): o.get_attr("value") for o in pre if o.get_name() == "frisk.fill"}
    if len(q_load) != 1 or len(pre) != 1 + len(fills):
        _fail("attention prologue must be the Q tile copy and fills")
    q_src, q_buf, q_org, q_do, _, _ = _tile_copy(q_load[0], ivs)

    gemms = [o for o in lops if o.get_name() == "frisk.gemm"]
    if len(gemms) != 2:
        _fail("the key-block loop must hold the score GEMM and the PV GEMM")
    g_s, g_o = (fr.GemmOp.from_operation(g) for g in gemms)
    s_acc, o_acc = g_s.get_matrix_C(), g_o.get_matrix_C()
    if g_s.get_matrix_A() != q_buf:
        _fail("the score GEMM must read the Q tile")
    if not gemms[0].get_attr("clear_accum") and fills.get(s_acc.id()) is None:
        _fail("scores must be cleared each key block")
    if gemms[1].get_attr("clear_accum") or fills.get(o_acc.id()) != 0.0:
        _fail("the output accumulator must be zero-filled once and accumulated")
    k_buf, k_trans = g_s.get_matrix_B(), not bool(gemms[0].get_attr("transB"))
    reds = [fr.ReduceOp.from_operation(o) for o in lops if o.get_name() == "frisk.reduce"]
    kinds = sorted(o.get_attr("kind") for o in lops if o.get_name() == "frisk.reduce")
    if kinds not in (["max"], ["add", "max"]):
        _fail("scores must be reduced by max (and optionally add) along the key axis")
    for r, o in zip(reds, [o for o in lops if o.get_name() == "frisk.reduce"]):
        if r.get_src_memref() != s_acc or r.get_reduce_dim() != 1 or o.get_attr("clear"):
            _fail("row statistics must merge the scores along dim 1 (clear = false)")
        init = fills.get(r.get_dst_memref().id())
        if init != (-math.inf if o.get_attr("kind") == "max" else 0.0):
            _fail("row maxima must start at -inf and row sums at 0")
    copies = [o for o in lops if o.get_name() == "frisk.copy"]
    p_buf = g_o.get_matrix_A()
    loads = {}
    cast_ok = False
    for cop in copies:
        src, dst, so, do, sext, dext = _tile_copy(cop, ivs)
        if src == s_acc and dst == p_buf:
            cast_ok = True
        else:
            loads[dst.id()] = (src, so)
    if not cast_ok:
        _fail("scores must be cast into the PV GEMM's P operand")
    if k_buf.id() not in loads or g_o.get_matrix_B().id() not in loads:
        _fail("K and V tiles must be loaded in the key-block loop")
    k_src, k_org = loads[k_buf.id()]
    v_src, v_org = loads[g_o.get_matrix_B().id()]
    # Epilogue: accumulator -> (optional Shared staging) -> O.
    src, dst, so, o_org, _, oext = _tile_copy(post[-1], ivs)
    stage = [o for o in post[:-1] if o.get_name() == "frisk.copy"]
    if len(post) - 1 != len(stage) or len(stage) > 1:
        _fail("attention epilogue must copy the accumulator into O")
    if stage:
        s_src, s_dst, *_ = _tile_copy(stage[0], ivs)
        if s_src != o_acc or s_dst != src:
            _fail("the staged epilogue must copy the accumulator into the staging tile")
    elif src != o_acc:
        _fail("the epilogue must store the output accumulator")
    idx = [_arg_index(v, entry) for v in (q_src, k_src, v_src, dst)]
    if None in idx:
        _fail("Q, K, V and O must be kernel arguments")
    shape = _shape(q_src)
    if len(shape) != 4:
        _fail("Q/K/V/O must be rank-4 [batch, heads, seq, head_dim] memrefs")
    B, H, S, D = shape
    bm = _shape(q_buf)[0]
    bn = _shape(s_acc)[1]
    k_shape = _shape(k_src)
    if k_shape != ([B, H, D, S] if k_trans else [B, H, S, D]) or _shape(v_src) != shape or \
            _shape(dst) != shape:
        _fail("K/V/O shapes disagree with Q")

    def check(org, seq_dim, per_trip_key, stride, name):
        c0, coef = org
        want = {pk[0]: [1 if d == 0 else 0 for d in range(4)],
                pk[1]: [1 if d == 1 else 0 for d in range(4)]}
        if c0 != [0, 0, 0, 0]:
            _fail(f"{name} tile origin must start at 0")
        for key in (pk[0], pk[1]):
            if coef.get(key) != want[key]:
                _fail(f"{name} tile must follow the batch and head grid axes")
        seq = coef.get(per_trip_key, [0] * 4)
        if seq != [stride if d == seq_dim else 0 for d in range(4)]:
            _fail(f"{name} tile sequence offset must advance by {stride}")
        others = set(coef) - {pk[0], pk[1], per_trip_key}
        if others:
            _fail(f"{name} tile depends on an unexpected index")

    check(q_org, 2, pk[2], bm, "Q")
    check(o_org, 2, pk[2], bm, "O")
    check(k_org, 3 if k_trans else 2, kkey, bn, "K")
    check(v_org, 2, kkey, bn, "V")
    if grid != [B, H, S // bm] or S % bm or ivs.ranges[kkey][2] * bn != S:
        _fail(f"grid {grid} / key loop do not cover B={B} H={H} S={S}")
    return AttnPlan(*idx, k_trans, B, H, S, D)


# ---------------------------------------------------------------------------
def tile_contract(bm: int, bn: int, bk: int, dtype: str, trans_a: bool, trans_b: bool,
                  threads: int, policy=None):
    """(contract, reason) of the workgroup tile product C[bm, bn] += op(A).op(B)
    (A, B tiles in Shared memory, f32 accumulator, `threads` lanes, warp
    `policy`): the `#frisk.mma_contract` layout inference binds for it, or
    (None, reason) when inference finds none."""
    return _tile_contract(bm, bn, bk, dtype, bool(trans_a), bool(trans_b), threads,
                          None if policy is None else str(policy), policy)


@lru_cache(maxsize=256)
def _tile_contract(bm, bn, bk, dtype, trans_a, trans_b, threads, policy_key, policy):
    try:
        from .common import utils
        s = utils.create_session()
        S = ir.MemorySpace.SHARED
        acc_t = "int32" if dtype == "int8" else "fp32"
        _, entry = s.new_kernel("tile", [
            s.memref_type([bk, bm] if trans_a else [bm, bk], dtype, space=S),
            s.memref_type([bn, bk] if trans_b else [bk, bn], dtype, space=S),
            s.memref_type([bm, bn], acc_t)])
        acc = s.alloc_buffer([bm, bn], acc_t)
        g = s.create_gemm(entry.get_argument(0), entry.get_argument(1), acc, trans_a=trans_a,
                          trans_b=trans_b, clear_accum=True, legacy_semantics="tensor_v1")
        if policy is not None:
            g.set_attr("policy", s.builder.get_gemm_warp_policy_attr(policy))
        g.set_attr("frisk.execution_threads", s.builder.get_int64_attr(threads))
        s.builder.create_copy_op(acc, entry.get_argument(2), [], [])
        fr.normalize_layout_ir(s.module, "gfx950")
        rep = fr.infer_layouts(s.module)
        if rep.get("status") != "materialized":
            raise ValueError(f"layout inference {rep.get('status')}: {rep.get('failure', '')}")
        found = [a for a in rep["assignments"] if a.startswith("mma#")]
        return found[0].split(": ", 1)[1], ""
    except (ValueError, RuntimeError) as e:  # reported as the reason; the GEMM still runs
        return None, f"no instruction contract: {e}"


def _device_cus() -> int:
    """Compute units of the current GPU (256, MI355X's count, without one)."""
    try:
        import torch
        if torch.cuda.is_available():
            return int(torch.cuda.get_device_properties(torch.cuda.current_device())
                       .multi_processor_count)
    except Exception:  # no torch / no device: plan for the MI355X
        pass
    return 256


_TYPES_SESSION = []  # one session kept alive: its context owns the types below


@lru_cache(maxsize=None)
def _type_of(elem: str):
    """An IR element type from its spelling, owned by a session that lives as
    long as the process."""
    from .common import utils
    if not _TYPES_SESSION:
        _TYPES_SESSION.append(utils.create_session())
    names = dict(_HELPER_NAMES, i32="int32")
    return _TYPES_SESSION[0]._as_type(names.get(elem, elem))


def _launch(p: "GemmPlan") -> dict:
    """The target's launch contract of the whole GEMM (with a workspace)."""
    a_ty, c_ty = (_type_of(e) for e in p.elems)
    return fr.gemm_launch_plan(p.m, p.n, p.k, a_ty, c_ty, p.trans_a, p.trans_b,
                               cus=_device_cus(), workspace=True)


def _bind_variant(p: "GemmPlan", tile) -> "GemmPlan":
    """Fill p.launch / contract / variant / layouts_match / mismatch: the
    kernel variant that executes the program's workgroup tile product (a
    tiled program), or the one the launch contract names for the whole GEMM
    (a whole-matrix program)."""
    try:
        p.launch = _launch(p)
    except ValueError as e:
        p.mismatch = f"no launch contract: {e}"
        return p
    p.swizzle_match = _swizzles_match(p)
    if tile is None:
        L = p.launch
        if L["kernel"] not in ("gemm_w4", "gemm_128"):
            # The small-M and generic kernels have no tile program: the
            # launch contract names them, and the library runs them.
            p.contract, p.layouts_match = L["contract"], True
            return p
        dname = _HELPER_NAMES.get(p.elems[0], p.elems[0])
        bt, (wm, wn) = L["tile"][0], L["wave_grid"]
        tile = (bt, bt, L["stage_bytes"] // _ESIZE.get(dname, 2), dname, p.policy, 64 * wm * wn)
    bm, bn, bk, dtype, policy, threads = tile
    p.contract, why = tile_contract(bm, bn, bk, dtype, p.trans_a, p.trans_b, threads, policy)
    if p.contract is not None:
        p.variant, why = variants.variant_for(p.contract, bm, bn, threads)
    if p.variant is not None:
        # The launch contract's K split, when it runs this very tile and grid.
        L = p.launch
        if L["kernel"] in ("gemm_w4", "gemm_128") and L["tile"] == [bm, bn] and \
                list(p.variant[1:]) == L["wave_grid"] and L["slices"] > 1:
            p.variant = tuple(p.variant) + (L["slices"],)
    p.layouts_match = p.variant is not None
    p.mismatch = why
    return p


def _swizzles_match(p: "GemmPlan") -> Optional[bool]:
    """Checks the MFMA kernel's LDS swizzles against the layout target's
    storage proposal (`F.frisk.lds_swizzle`, the swizzle inference gives a
    Shared tile read by MFMA fragments) for the kernel's K-major stage rows.
    The M/N-major tiles are read by transposing loads, which the proposer
    does not model; they are not compared."""
    L = p.launch
    if L is None or L["kernel"] not in ("gemm_w4", "gemm_128"):
        return None
    proposal = fr.lds_swizzle(L["stage_bytes"], 32).formula
    kmajor = [L["lds_swizzle_a"]] if not p.trans_a else []
    kmajor += [L["lds_swizzle_b"]] if p.trans_b else []
    return all(sw == proposal for sw in kmajor) if kmajor else None


def _checked_variant(p: "GemmPlan", a, b, c):
    """p.variant if the C-ABI runs it on these tensors, else None (the
    library's own choice then runs, and p.mismatch / layouts_match say so)."""
    from . import runtime as rt
    if p.variant is None:
        return None
    try:
        rt.gemm_plan(a, b, c, trans_a=p.trans_a, trans_b=p.trans_b, variant=p.variant)
    except ValueError as e:
        p.mismatch = f"variant {p.variant} does not run on these tensors ({e}); the library's own " \
                     "choice runs"
        p.layouts_match = False
        return None
    return p.variant


def plan(module, kernel: str):
    """Recognise kernel `kernel` of `module`: a GemmPlan, an AttnPlan or a
    tileprog.OpsPlan (fill / copy / reduce programs).  A GemmPlan carries the
    tile product's instruction contract and the kernel variant it selects."""
    k = module.get_kernel(kernel)
    if k is None:
        raise ValueError(f"execute: module has no kernel @{kernel}")
    if not k.verify():
        raise ValueError(f"execute: kernel @{kernel} does not verify: {k.verify_diagnostic()}")
    entry = k.get_region(0).front()
    ops = _body_ops(entry)
    reasons = []
    for recognise in (_gemm_whole, _gemm_tiled, _attention, tileprog.plan_whole,
                      tileprog.plan_tiled):
        try:
            p = recognise(ops, entry)
            return _bind_variant(p, p.tile) if isinstance(p, GemmPlan) else p
        except (_Reject, tileprog.Reject) as e:
            reasons.append(f"{recognise.__name__.lstrip('_')}: {e}")
    raise ValueError(f"execute: kernel @{kernel} is not a recognised GEMM, attention or tile-op "
                     "program ("
                     + "; ".join(reasons) + ")")


_TORCH_DTYPES = {"f16": "float16", "bf16": "bfloat16", "f32": "float32", "f8E4M3FN": "float8_e4m3fn",
                 "i8": "int8", "i32": "int32", "f64": "float64"}


def _check_tensor(t, value, name):
    import torch
    shape = _shape(value)
    want = _TORCH_DTYPES.get(_elem(value))
    if want is None or t.dtype != getattr(torch, want):
        raise ValueError(f"execute: {name} must be {_elem(value)} (got {t.dtype})")
    if list(t.shape) != shape:
        raise ValueError(f"execute: {name} must have shape {shape} (got {list(t.shape)})")
    if not t.is_cuda:
        raise ValueError(f"execute: {name} must be a device tensor")


def execute(module, kernel: str, tensors: Sequence, *, stream=None, causal: bool = False,
            sm_scale: Optional[float] = None, scale_a: float = 1.0, scale_b: float = 1.0,
            require_layout_match: bool = False):
    """Run kernel `kernel` of `module` on `tensors` (one per kernel argument).
    With require_layout_match a GEMM whose contracts no kernel runs raises
    ValueError instead of running the library's own choice."""
    from . import runtime as rt
    p = plan(module, kernel)
    k = module.get_kernel(kernel)
    args = [k.arg(i) for i in range(k.get_num_arguments())]
    if len(tensors) != len(args):
        raise ValueError(f"execute: @{kernel} takes {len(args)} tensors, got {len(tensors)}")
    for i, (t, a) in enumerate(zip(tensors, args)):
        _check_tensor(t, a, f"argument {i}")
    if isinstance(p, tileprog.OpsPlan):
        return tileprog.run(p, tensors, stream=stream)
    if isinstance(p, GemmPlan):
        a, b, c = tensors[p.a], tensors[p.b], tensors[p.c]
        variant = _checked_variant(p, a, b, c)
        if require_layout_match and not p.layouts_match:
            raise ValueError(f"execute: no kernel runs the contracts of @{kernel} ({p.mismatch})")
        return rt.gemm(a, b, c, trans_a=p.trans_a, trans_b=p.trans_b, clear_accum=p.clear_accum,
                       scale_a=scale_a, scale_b=scale_b, stream=stream, variant=variant)
    q, kk, v, o = (tensors[i] for i in (p.q, p.k, p.v, p.o))
    # A K stored [B, H, D, S] (the reference's FA tile program) is read in
    # place by the kernel's transposed-K variant; the waves per workgroup
    # come from the attention launch contract.
    waves = fr.attention_launch_plan(p.batch * p.heads, p.seq, p.head_dim, causal,
                                     _device_cus())["waves"]
    p.waves = {"causal" if causal else "full": waves}
    return rt.attn_fwd(q, kk, v, o, causal=causal, sm_scale=sm_scale, stream=stream,
                       k_transposed=p.k_transposed, waves=waves)
