"""Reduction, fill and copy execution packets on the CPU: what plan_packet
makes of them, and that the leaf order it derives from the fibers
reproduces the packet's own canonical trees (ReductionLayoutProof.cpp:
108-140) on association-sensitive data."""
import numpy as np
import pytest

import frisk_amd as F
from frisk_amd.packet import leaf_order_of
from oracle import tileops as T
from tests import programs as P


def fiber_tree_reference(packet, x, kind, dtype):
    """The packet's contract computed from the packet alone: for each output,
    the fiber's leaves (carrier -> element through the source layout's
    logical enumeration) combined by the canonical tree."""
    ops = packet["operations"]
    red = next(o for o in ops if o["name"] == "frisk.reduce_tensor")
    load = next(o for o in ops if o["name"] == "frisk.tile_load")
    src = next(v for v in packet["values"] if v["id"] == load["results"][0])
    logical = src["distributed"]["logical"]
    flat = np.asarray(x, dtype=np.float32).reshape(-1)
    leaves = np.array([[flat[logical[c]] for c in fiber] for fiber in red["fibers"]],
                      dtype=np.float32)
    return T.canonical_tree(T.KINDS[kind], dtype, leaves)


@pytest.mark.parametrize("dim", [1, 0])
@pytest.mark.parametrize("shape,threads", [((64, 64), 128), ((32, 16), 64), ((128, 32), 256)])
def test_reduce_packet_plan_and_leaf_order(dim, shape, threads):
    R, C = shape
    pk = P.exported_packet(P.single_tile_reduce(R, C, kind="add", dim=dim, threads=threads))
    plan = F.plan_packet(pk)
    assert plan["kind"] == "reduce" and plan["dim"] == dim and plan["init"] is None
    assert (plan["src"], plan["dst"]) == (0, 1)
    rng = np.random.default_rng(R * C + dim)
    x = (rng.standard_normal((R, C)) * np.exp2(rng.integers(-20, 21, (R, C)))).astype(np.float32)
    want = fiber_tree_reference(pk, x, "add", "f32")
    got = T.reduce(x, "sum", dim, "f32", leaf_order=plan["leaf_order"])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_column_sum_packet_needs_its_permuted_order():
    """The solver's 64x64 layout walks rows through registers first, so the
    column-sum fibers are not in ascending row order; ascending order gives
    different sums on sensitive data."""
    pk = P.exported_packet(P.single_tile_reduce(64, 64, kind="add", dim=0, threads=128))
    order = F.plan_packet(pk)["leaf_order"]
    assert order is not None and sorted(order) == list(range(6)) and order != list(range(6))
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 64)) * np.exp2(rng.integers(-20, 21, (64, 64)))).astype(np.float32)
    want = fiber_tree_reference(pk, x, "add", "f32")
    asc = T.reduce(x, "sum", 0, "f32")
    assert not np.array_equal(asc.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind,init", [("max", float("-inf")), ("add", 0.5), ("min", 3.0)])
def test_merge_packet_carries_the_initial_value(kind, init):
    pk = P.exported_packet(P.single_tile_reduce(64, 64, kind=kind, init=init))
    plan = F.plan_packet(pk)
    assert plan["kind"] == "reduce" and plan["init"] == init
    assert plan["reduce"] == {"add": "sum"}.get(kind, kind)


def test_fill_and_copy_packets():
    plan = F.plan_packet(P.exported_packet(P.single_tile_fill(64, 64, value=-2.25)))
    assert plan["kind"] == "fill" and plan["value"] == -2.25 and plan["dst"] == 0
    plan = F.plan_packet(P.exported_packet(P.single_tile_copy(64, 64)))
    assert plan["kind"] == "copy" and (plan["src"], plan["dst"]) == (0, 1)


def test_leaf_order_rejects_non_permutations():
    logical = list(range(16))  # carrier c holds element c of a 4x4 tile
    assert leaf_order_of([[0, 4, 8, 12]], logical, [4, 4], 0) is None
    assert leaf_order_of([[0, 8, 4, 12]], logical, [4, 4], 0) == [1, 0]
    with pytest.raises(ValueError, match="not a permutation"):
        leaf_order_of([[0, 12, 4, 8]], logical, [4, 4], 0)
    with pytest.raises(ValueError, match="different leaf orders"):
        leaf_order_of([[0, 4, 8, 12], [1, 9, 5, 13]], logical, [4, 4], 0)
    with pytest.raises(ValueError, match="power-of-two"):
        leaf_order_of([[0, 4, 8]], logical, [3, 4], 0)
