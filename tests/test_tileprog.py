"""Plans of fill / copy / reduce tile programs (frisk_amd/tileprog.py), on the
CPU: which launches a program lifts to, and the programs that must be
rejected because their tiles do not partition the tensors or a reduction
does not lie inside one tile."""
import re

import pytest

import frisk_amd as F
from frisk_amd import executor as E
from tests import programs as P


def kernel_name(s):
    return re.search(r"frisk.kernel @(\w+)", str(s.module)).group(1)


def plan_of(built):
    s, _ = built
    return E.plan(s.module, kernel_name(s))


def resolved(p, key):
    b = p.bufs[key]
    while b.alias is not None:
        b = p.bufs[b.alias]
    return b.key


def launches(p):
    out = []
    for st in p.steps:
        if st[0] == "fill":
            out.append(("fill", resolved(p, st[1])))
        elif st[0] == "gemm":
            out.append(("gemm",) + tuple(resolved(p, k) for k in st[1:4]))
        else:
            out.append((st[0], resolved(p, st[1]), resolved(p, st[2])) + tuple(st[3:]))
    return out


def test_row_reduce_is_one_reduction_from_argument_to_argument():
    p = plan_of(P.row_reduce(256, 64, kind="max"))
    assert launches(p) == [("reduce", "arg0", "arg1", "max", 1, True)]
    assert p.bufs["tile0"].shape == [256, 64] and p.bufs["tile1"].shape == [256]


def test_merge_reduction_fills_then_merges_in_place():
    p = plan_of(P.row_reduce(128, 32, kind="add", init=0.0))
    assert launches(p) == [("fill", "arg1"), ("reduce", "arg0", "arg1", "add", 1, False)]


def test_column_strips_reduce_along_dim0():
    p = plan_of(P.col_reduce_tiles(100, 256, BC=64))
    assert launches(p) == [("reduce", "arg0", "arg1", "add", 0, True)]


@pytest.mark.parametrize("staged", [False, True])
def test_cast_is_one_converting_copy(staged):
    p = plan_of(P.tiled_cast(128, 256, staged=staged))
    assert launches(p) == [("copy", "arg0", "arg1")]


def test_fill_program_fills_the_argument():
    p = plan_of(P.tiled_fill(64, 128, 1.5))
    assert launches(p) == [("fill", "arg0")] and p.steps[0][2] == 1.5


def test_whole_tensor_sequence_keeps_its_temporary():
    p = plan_of(P.gemm_then_cast(64, 64, 64))
    assert p.form == "whole"
    assert launches(p) == [("fill", "tmp0"), ("gemm", "arg0", "arg1", "tmp0"),
                           ("copy", "tmp0", "arg2")]
    assert p.bufs["tmp0"].shape == [64, 64] and p.bufs["tmp0"].elem == "f32"


def custom(R=256, C=64, grid=(4,), tile=(64, 64), xmap=None, ymap=None, dim=1, out_shape=None,
           store_ivs=None, inplace=False):
    """A row-reduction program with every placement under the test's control."""
    s = F.create_session()
    b = s.builder
    G = F.MemorySpace.GLOBAL
    out_shape = out_shape or [R]
    args = [s.memref_type([R, C], "fp32", space=G)]
    if not inplace:
        args.append(s.memref_type(out_shape, "fp32", space=G))
    kernel, entry = s.new_kernel("custom", args)
    X = entry.get_argument(0)
    Y = X if inplace else entry.get_argument(1)
    par = b.create_parallel_op(list(grid), 128)
    b.set_insertion_point_to_start(par.add_entry_block())
    ivs = list(par.get_ivs())
    t = s.alloc_buffer(list(tile), "fp32")
    r = s.alloc_buffer([tile[1 - dim]], "fp32")
    ctx = s.context
    d = [b.get_affine_dim_expr(i) for i in range(len(grid))]
    zero = b.get_affine_constant_expr(0)
    empty = b.get_empty_affine_map()
    xm = F.AffineMap.get(len(grid), 0, xmap(d, zero), ctx)
    b.create_copy_op(X, t, ivs, [], xm, empty)
    b.create_reduce_op(t, r, "max", dim, True)
    if inplace:
        b.create_copy_op(t, Y, [], ivs, empty, xm, list(tile), list(tile))
    else:
        ym = F.AffineMap.get(len(store_ivs or ivs), 0, ymap(d, zero), ctx)
        b.create_copy_op(r, Y, [], store_ivs or ivs, empty, ym, [tile[1 - dim]], [tile[1 - dim]])
    return s, kernel


def test_custom_baseline_is_accepted():
    p = plan_of(custom(xmap=lambda d, z: [d[0] * 64, z], ymap=lambda d, z: [d[0] * 64]))
    assert launches(p) == [("reduce", "arg0", "arg1", "max", 1, True)]


@pytest.mark.parametrize("kw,msg", [
    (dict(grid=(4, 2), tile=(64, 32), xmap=lambda d, z: [d[0] * 64, d[1] * 32],
          ymap=lambda d, z: [d[0] * 64]), "store must use every grid axis"),
    (dict(xmap=lambda d, z: [d[0] * 32, z], ymap=lambda d, z: [d[0] * 64]),
     "advance by the tile extent"),
    (dict(grid=(3,), xmap=lambda d, z: [d[0] * 64, z], ymap=lambda d, z: [d[0] * 64]),
     "cover 256"),
    (dict(tile=(64, 32), xmap=lambda d, z: [d[0] * 64, z], ymap=lambda d, z: [d[0] * 64]),
     "must span it"),
    (dict(grid=(4, 2), xmap=lambda d, z: [d[0] * 64, z], ymap=lambda d, z: [d[0] * 64],
          out_shape=[256]), "store must use every grid axis"),
    (dict(xmap=lambda d, z: [d[0] * 64 + 64, z], ymap=lambda d, z: [d[0] * 64]),
     "origin must be 0"),
    (dict(xmap=lambda d, z: [d[0] * 64, z], inplace=True), "both loaded and stored"),
])
def test_programs_that_do_not_partition_are_rejected(kw, msg):
    s, _ = custom(**kw)
    with pytest.raises(ValueError, match=msg):
        E.plan(s.module, "custom")


def test_unsupported_whole_op_is_named():
    s = F.create_session()
    G = F.MemorySpace.GLOBAL
    kernel, entry = s.new_kernel("blk", [s.memref_type([64, 64], "fp32", space=G)])
    s.builder.create_block_op([64, 64], lambda b2, ivs: None)
    with pytest.raises(ValueError, match="frisk.block is not a whole-tensor"):
        E.plan(s.module, "blk")
