"""Tile programs built from fill / copy / reduce (and GEMM) steps, run as
whole-tensor launches of frisk_fill, frisk_copy, frisk_reduce and frisk_gemm.

Two forms are recognised (the ops of include/Dialect/Frisk/IR/FriskOps.td:
gemm :252-292, alloc_buffer :295-348, copy :351-397, fill :400-422, reduce
:425-453):

* whole-tensor: the kernel body is a sequence of frisk.fill, whole-buffer
  frisk.copy (no indices or maps, equal shapes; the element type may change),
  frisk.reduce and frisk.gemm on kernel arguments and on Global buffers
  allocated at the top of the body.  Each op becomes one launch, in order.
* tiled: one frisk.parallel whose body allocates Local/Shared tiles, loads
  them from kernel arguments with frisk.copy at affine tile origins, applies
  fill / copy / reduce to the tiles and stores tiles back with frisk.copy.
  Every global access must place its tile at (extent * grid index) along the
  dimensions that a grid axis walks and at 0 along the others, with grid x
  extent equal to the argument's extent, so that the tiles partition the
  argument; a reduction must span its tile's whole reduced dimension, and
  every store must use every grid axis (each element is written once).
  Under those conditions each tile op equals the same op on the whole
  tensors assembled from the tiles ("lifting"), which is what runs: a tile
  buffer becomes a whole tensor of grid x tile shape.  Loads of an argument
  that the program never overwrites alias it; a tile that is only computed
  and then stored in the argument's dtype is computed in place.

Reductions keep their canonical_fiber_tree_v1 order under lifting because the
tile spans the whole reduced extent.  Anything else raises ValueError naming
the first mismatch; there is no CPU path.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

from . import _ir

ir = _ir()
fr = ir.frisk

_ELEM = {"f16": "float16", "bf16": "bfloat16", "f32": "float32", "f8E4M3FN": "float8_e4m3fn",
         "i8": "int8", "i32": "int32", "f64": "float64"}


class Reject(ValueError):
    pass


def _fail(msg: str):
    raise Reject(msg)


@dataclass
class Buf:
    """A whole tensor of the lifted program: a kernel argument or a temporary."""
    key: str
    shape: list
    elem: str
    arg: Optional[int] = None      # kernel argument index when it is one
    alias: Optional[str] = None    # buffer whose storage this one shares


@dataclass
class OpsPlan:
    bufs: dict = field(default_factory=dict)    # key -> Buf
    steps: list = field(default_factory=list)   # (op, ...) over buffer keys
    form: str = "whole"


def _body_ops(block) -> list:
    return [op for op in block.get_operations() if op.get_name() != "frisk.end"]


def _shape(value):
    return list(value.get_type().get_shape())


def _elem(value):
    return str(value.get_type().get_element_ty())


def _is_arg(value, entry) -> Optional[int]:
    if not hasattr(value, "get_owner") or value.get_owner().id() != entry.id():
        return None
    return value.get_arg_number()


def _reduce_attrs(op):
    kind = op.get_attr("kind")
    if kind not in ("add", "sum", "max", "min"):
        _fail(f"reduce kind {kind!r} is not add / max / min")
    return kind, int(op.get_attr("dim")), bool(op.get_attr("clear"))


def _check_reduce_shapes(src_shape, dst_shape, dim):
    if len(src_shape) != 2 or dim not in (0, 1) or dst_shape != [src_shape[1 - dim]]:
        _fail(f"reduce of {src_shape} along {dim} into {dst_shape}: needs a rank-2 source "
              "and the rank-1 destination of the kept dimension")


# ---------------------------------------------------------------------------
# Whole-tensor sequences
# ---------------------------------------------------------------------------
def plan_whole(ops, entry) -> OpsPlan:
    p = OpsPlan(form="whole")
    names = {}

    def buf(value):
        i = _is_arg(value, entry)
        if i is not None:
            key = f"arg{i}"
            if key not in p.bufs:
                p.bufs[key] = Buf(key, _shape(value), _elem(value), arg=i)
            return key
        k = names.get(value.id())
        if k is None:
            _fail("operands must be kernel arguments or top-level Global buffers")
        return k

    saw_work = False
    for op in ops:
        name = op.get_name()
        if name == "frisk.alloc_buffer":
            v = op.get_result(0)
            if v.get_type().get_memory_space() != ir.MemorySpace.GLOBAL:
                _fail("top-level buffers of a whole-tensor program must be Global")
            key = f"tmp{len(names)}"
            names[v.id()] = key
            p.bufs[key] = Buf(key, _shape(v), _elem(v))
        elif name == "frisk.fill":
            p.steps.append(("fill", buf(op.get_operand(0)), float(op.get_attr("value"))))
            saw_work = True
        elif name == "frisk.copy":
            cp = fr.CopyOp.from_operation(op)
            if list(cp.get_src_indices()) or list(cp.get_dst_indices()) or \
                    cp.get_src_affine_map().get_num_results() or cp.get_dst_affine_map().get_num_results():
                _fail("whole-tensor copies take no indices or maps")
            s, d = buf(cp.get_src_memref()), buf(cp.get_dst_memref())
            if p.bufs[s].shape != p.bufs[d].shape:
                _fail(f"copy {p.bufs[s].shape} -> {p.bufs[d].shape}: shapes differ")
            p.steps.append(("copy", s, d))
            saw_work = True
        elif name == "frisk.reduce":
            r = fr.ReduceOp.from_operation(op)
            s, d = buf(r.get_src_memref()), buf(r.get_dst_memref())
            kind, dim, clear = _reduce_attrs(op)
            _check_reduce_shapes(p.bufs[s].shape, p.bufs[d].shape, dim)
            p.steps.append(("reduce", s, d, kind, dim, clear))
            saw_work = True
        elif name == "frisk.gemm":
            g = fr.GemmOp.from_operation(op)
            a, b, c = (buf(v) for v in (g.get_matrix_A(), g.get_matrix_B(), g.get_matrix_C()))
            p.steps.append(("gemm", a, b, c, bool(op.get_attr("transA")),
                            bool(op.get_attr("transB")), bool(op.get_attr("clear_accum"))))
            saw_work = True
        else:
            _fail(f"{name} is not a whole-tensor fill / copy / reduce / gemm step")
    if not saw_work:
        _fail("no fill / copy / reduce / gemm step")
    for b in p.bufs.values():
        if len(b.shape) > 2:
            _fail(f"tile ops here take rank-1 or rank-2 tensors (got {b.shape})")
    return p


# ---------------------------------------------------------------------------
# Tiled programs
# ---------------------------------------------------------------------------
def _affine_origin(amap, indices, ivs, rank):
    """(constant origin, {grid axis: per-index offset vector}) of a copy side."""
    if amap.get_num_results() == 0:
        if indices:
            _fail("copy indices without a map")
        return [0] * rank, {}
    if amap.get_num_results() != rank or amap.get_num_symbols():
        _fail(f"copy map {amap} must give one offset per dimension without symbols")
    for e in amap.get_results():
        if not e.is_pure_affine():
            _fail(f"copy map result {e} is not pure affine")
    axes = []
    for v in indices:
        if not hasattr(v, "get_owner") or v.get_owner().id() != ivs["block"]:
            _fail("copy indices must be the parallel's induction variables")
        axes.append(v.get_arg_number())
    base = [0] * len(axes)
    c0 = amap.evaluate(base)
    coef = {}
    for k in set(axes):
        pt = [1 if axes[i] == k else 0 for i in range(len(axes))]
        d = [x - y for x, y in zip(amap.evaluate(pt), c0)]
        # linear in the index: the offset at 2 must be twice the offset at 1
        pt2 = [2 if axes[i] == k else 0 for i in range(len(axes))]
        d2 = [x - y for x, y in zip(amap.evaluate(pt2), c0)]
        if d2 != [2 * x for x in d]:
            _fail(f"copy map {amap} is not linear in the grid index")
        if any(d):
            coef[k] = d
    return c0, coef


def _tile_mapping(origin, tile_shape, global_shape, grid, what):
    """dim -> grid axis (or None) for a tile placed at `origin` in a global
    tensor; checks that the tiles partition the tensor."""
    c0, coef = origin
    if len(tile_shape) != len(global_shape):
        _fail(f"{what}: tile rank {len(tile_shape)} differs from the argument's {len(global_shape)}")
    if any(c0):
        _fail(f"{what}: tile origin must be 0 at grid index 0 (got {c0})")
    mapping = []
    used = set()
    for d, (t, g) in enumerate(zip(tile_shape, global_shape)):
        axes = [k for k, vec in coef.items() if vec[d]]
        if not axes:
            if t != g:
                _fail(f"{what}: dimension {d} is not walked by the grid, so the tile must span "
                      f"it ({t} != {g})")
            mapping.append(None)
            continue
        if len(axes) != 1:
            _fail(f"{what}: dimension {d} depends on several grid axes")
        k = axes[0]
        if k in used:
            _fail(f"{what}: grid axis {k} moves more than one dimension")
        used.add(k)
        if coef[k][d] != t or grid[k] * t != g:
            _fail(f"{what}: dimension {d} must advance by the tile extent {t} per index of grid "
                  f"axis {k} and cover {g} (grid {grid[k]})")
        mapping.append(k)
    return mapping


def plan_tiled(ops, entry) -> OpsPlan:
    if len(ops) != 1 or ops[0].get_name() != "frisk.parallel":
        _fail("not a tiled tile-op program (expected one frisk.parallel)")
    par = fr.ParallelOp.from_operation(ops[0])
    grid = list(par.get_grid())
    block = par.get_region(0).front()
    ivs = {"block": block.id()}
    body = _body_ops(block)
    p = OpsPlan(form="tiled")
    tiles = {}      # value id -> key
    tile_shape = {}
    mapping = {}    # key -> list(dim -> grid axis or None)
    steps = []      # (op, ...) with tile keys / arg keys
    read_args, written_args = set(), set()

    def argbuf(value):
        i = _is_arg(value, entry)
        if i is None:
            return None
        key = f"arg{i}"
        if key not in p.bufs:
            p.bufs[key] = Buf(key, _shape(value), _elem(value), arg=i)
        return key

    def tile(value):
        k = tiles.get(value.id())
        if k is None:
            _fail("tile operands must be buffers allocated in the parallel body")
        return k

    def set_map(key, m, what):
        if key in mapping and mapping[key] != m:
            _fail(f"{what}: tile {key} is used with two different grid placements")
        mapping[key] = m

    for op in body:
        name = op.get_name()
        if name == "frisk.alloc_buffer":
            v = op.get_result(0)
            if v.get_type().get_memory_space() == ir.MemorySpace.GLOBAL:
                _fail("buffers inside the parallel must be Local or Shared tiles")
            key = f"tile{len(tiles)}"
            tiles[v.id()] = key
            tile_shape[key] = _shape(v)
            p.bufs[key] = Buf(key, None, _elem(v))
        elif name == "frisk.copy":
            cp = fr.CopyOp.from_operation(op)
            src, dst = cp.get_src_memref(), cp.get_dst_memref()
            sa, da = argbuf(src), argbuf(dst)
            if sa and da:
                _fail("a copy between two kernel arguments inside the parallel")
            if sa or da:  # load or store
                g, t = (src, dst) if sa else (dst, src)
                tk = tile(t)
                tmap = cp.get_dst_affine_map() if sa else cp.get_src_affine_map()
                tidx = list(cp.get_dst_indices()) if sa else list(cp.get_src_indices())
                if tmap.get_num_results() or tidx:
                    _fail("the tile side of a load / store is the whole tile")
                gmap = cp.get_src_affine_map() if sa else cp.get_dst_affine_map()
                gidx = list(cp.get_src_indices()) if sa else list(cp.get_dst_indices())
                ext = list(cp.get_src_extents()) if sa else list(cp.get_dst_extents())
                if ext and ext != tile_shape[tk]:
                    _fail(f"copy extents {ext} differ from the tile {tile_shape[tk]}")
                what = "load" if sa else "store"
                origin = _affine_origin(gmap, gidx, ivs, len(_shape(g)))
                m = _tile_mapping(origin, tile_shape[tk], _shape(g), grid, what)
                if da and any(grid[k] > 1 and k not in m for k in range(len(grid))):
                    _fail("a store must use every grid axis, or several tiles write one place")
                set_map(tk, m, what)
                if sa:
                    read_args.add(sa)
                    steps.append(("load", sa, tk))
                else:
                    written_args.add(da)
                    steps.append(("store", tk, da))
            else:
                s, d = tile(src), tile(dst)
                if tile_shape[s] != tile_shape[d]:
                    _fail(f"tile copy {tile_shape[s]} -> {tile_shape[d]}: shapes differ")
                if list(cp.get_src_indices()) or list(cp.get_dst_indices()) or \
                        cp.get_src_affine_map().get_num_results() or cp.get_dst_affine_map().get_num_results():
                    _fail("tile-to-tile copies take no indices or maps")
                steps.append(("copy", s, d))
        elif name == "frisk.fill":
            v = op.get_operand(0)
            if argbuf(v):
                _fail("fill of a kernel argument inside the parallel")
            steps.append(("fill", tile(v), float(op.get_attr("value"))))
        elif name == "frisk.reduce":
            r = fr.ReduceOp.from_operation(op)
            s, d = tile(r.get_src_memref()), tile(r.get_dst_memref())
            kind, dim, clear = _reduce_attrs(op)
            _check_reduce_shapes(tile_shape[s], tile_shape[d], dim)
            steps.append(("reduce", s, d, kind, dim, clear))
        else:
            _fail(f"{name} is not a tile fill / copy / reduce step")
    if not any(s[0] == "store" for s in steps):
        _fail("the program stores nothing")
    if read_args & written_args:
        _fail("an argument that is both loaded and stored (in-place tile programs are not lifted)")

    # Placements of tiles that touch no argument: propagate through copies
    # and reductions until nothing changes.
    changed = True
    while changed:
        changed = False
        for st in steps:
            if st[0] == "copy":
                s, d = st[1], st[2]
                for a, b in ((s, d), (d, s)):
                    if a in mapping and b not in mapping:
                        mapping[b] = mapping[a]
                        changed = True
                    elif a in mapping and b in mapping and mapping[a] != mapping[b]:
                        _fail(f"tile copy between different grid placements ({a}, {b})")
            elif st[0] == "reduce":
                s, d, dim = st[1], st[2], st[4]
                if s in mapping:
                    if mapping[s][dim] is not None:
                        _fail("a reduced dimension must lie inside one tile (the grid walks it)")
                    want = [x for i, x in enumerate(mapping[s]) if i != dim]
                    if d not in mapping:
                        mapping[d] = want
                        changed = True
                    elif mapping[d] != want:
                        _fail("reduction result placed differently from its source")
    def touches(st, key):
        return st[1] == key if st[0] == "fill" else key in st[1:3]

    for key in tile_shape:
        if key not in mapping:
            if any(touches(st, key) for st in steps):
                _fail(f"tile {key} is never placed on the grid (it neither comes from nor reaches "
                      "a kernel argument)")
            continue
        p.bufs[key].shape = [t * (grid[k] if k is not None else 1)
                             for t, k in zip(tile_shape[key], mapping[key])]
    for b in p.bufs.values():
        if b.shape is not None and len(b.shape) > 2:
            _fail(f"tile ops here take rank-1 or rank-2 tensors (got {b.shape})")

    # Storage: loads alias their argument when the tile is never written
    # afterwards and keeps its dtype; a tile that ends in exactly one store,
    # in the argument's dtype, and is read by nothing else is computed in
    # place in the argument.
    def written(st, key):
        return {"load": st[2], "fill": st[1], "copy": st[2], "reduce": st[2]}.get(st[0]) == key

    def read(st, key):
        if st[0] in ("copy", "reduce", "store") and st[1] == key:
            return True
        return st[0] == "reduce" and st[2] == key and not st[5]  # merge reads the old value

    out = []
    for st in steps:
        if st[0] == "load":
            a, t = st[1], st[2]
            if p.bufs[a].elem == p.bufs[t].elem and sum(written(x, t) for x in steps) == 1:
                p.bufs[t].alias = a
                continue
            out.append(("copy", a, t))
        elif st[0] == "store":
            t, a = st[1], st[2]
            stores = [x for x in steps if x[0] == "store" and x[1] == t]
            others = [x for x in steps if read(x, t) and x[0] != "store"
                      and not (x[0] == "reduce" and x[2] == t)]
            last = max(i for i, x in enumerate(steps) if touches(x, t))
            if p.bufs[t].alias is None and p.bufs[t].elem == p.bufs[a].elem and len(stores) == 1 \
                    and not others and steps.index(st) == last:
                p.bufs[t].alias = a
                continue
            out.append(("copy", t, a))
        else:
            out.append(st)
    p.steps = out
    return p


# ---------------------------------------------------------------------------
# Execution
# ---------------------------------------------------------------------------
def run(p: OpsPlan, tensors, stream=None):
    """Launch the plan's steps on the GPU, in order, on `stream`."""
    import torch
    from . import runtime as rt
    store = {}

    def resolve(key):
        b = p.bufs[key]
        while b.alias is not None:
            b = p.bufs[b.alias]
        if b.arg is not None:
            return tensors[b.arg]
        if b.key not in store:
            store[b.key] = torch.empty(b.shape, dtype=getattr(torch, _ELEM[b.elem]), device="cuda")
        return store[b.key]

    for st in p.steps:
        op = st[0]
        if op == "fill":
            rt.fill(resolve(st[1]), st[2], stream=stream)
        elif op == "copy":
            src, dst = resolve(st[1]), resolve(st[2])
            if src.data_ptr() != dst.data_ptr():
                rt.copy(src, dst, stream=stream)
        elif op == "reduce":
            rt.reduce(resolve(st[1]), resolve(st[2]), st[3], axis=st[4], clear=st[5], stream=stream)
        elif op == "gemm":
            rt.gemm(resolve(st[1]), resolve(st[2]), resolve(st[3]), trans_a=st[4], trans_b=st[5],
                    clear_accum=st[6], stream=stream)
        else:  # pragma: no cover - plans only hold the ops above
            raise AssertionError(op)
    return p
