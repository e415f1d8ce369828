"""Execution-packet consumer: run a packet written by frisk.export_execution
with this library's HIP kernels.

The reference executes its packets out of process, by generating Triton for
an H100 (benchmark/layout/execution/run_execution.py:23-95, packet format
lib/Conversion/FriskLayoutToGPU/ExportExecution.cpp:46-295).  Here the
packet's operation list is matched against the two tile programs the
library implements and dispatched through the C-ABI:

* GEMM: frisk.mma of two LDS/global tiles that frisk.copy filled from kernel
  arguments, then frisk.tile_store of the result -> frisk_gemm;
* attention: Q.K^T, scale, row max, exp, row sum, divide, truncate, P.V,
  store (the program of test/Transforms/attention-layout.mlir) ->
  frisk_attn_fwd with the packet's scale;
* reduction: frisk.tile_load, frisk.reduce_tensor (sum/max/min along one
  dim), optionally merged with a constant by arith.addf / maximumf /
  minimumf, frisk.tile_store -> frisk_fill of the constant and frisk_reduce.
  The packet's fibers fix the order of each sum
  (ReductionLayoutProof.cpp:108-140: an output's distinct inputs sorted by
  carrier, paired level by level); that order is read back from the fibers
  and the source layout's carrier enumeration and passed to frisk_reduce as
  its leaf order, so the sums are bit-exact with the packet's contract;
* fill: a splat constant stored by frisk.tile_store -> frisk_fill;
* copy: frisk.tile_load then frisk.tile_store -> frisk_copy.

The packet's distributed layouts describe how the solver would place the
tile; the kernels use their own fixed layouts, and `plan_packet` reports
whether the two agree (for attention the kernel computes S^T = K.Q^T with
32x32x16 MFMAs and queries on lanes; see frisk_amd/csrc/attn.h).
"""
from __future__ import annotations

import json
import re

from . import _ir, variants

__all__ = ["plan_packet", "execute_packet"]

_TRANSPARENT = {"memref.alloc", "frisk.layout_view", "frisk.copy", "arith.constant",
                "tensor.empty", "frisk.end", "frisk.kernel", "frisk.parallel",
                "frisk.convert_layout", "builtin.module"}
_ATTENTION = ["frisk.mma", "arith.mulf", "frisk.reduce_tensor", "linalg.broadcast", "arith.subf",
              "math.exp", "frisk.reduce_tensor", "linalg.broadcast", "arith.divf", "arith.truncf",
              "frisk.mma", "frisk.tile_store"]


def _load(packet) -> dict:
    pk = json.loads(packet) if isinstance(packet, (str, bytes)) else packet
    if not isinstance(pk, dict) or pk.get("schema_version") != 1 or pk.get("target") != "gfx950":
        raise ValueError("execution packet: expected schema_version 1 for target gfx950")
    return pk


def _splat(text: str) -> float:
    """Value of a splat constant: `dense<1.5> : ...`, or a hex bit pattern of
    the element type (`dense<0xFF800000> : tensor<64xf32>`), the form used for
    values without an exact decimal spelling such as infinities."""
    m = re.match(r"dense<([-+0-9.eEinfa]+)>", text or "")
    if m:
        return float(m.group(1))
    m = re.match(r"dense<0x([0-9A-Fa-f]+)>\s*:\s*\w+<(?:\d+x)*(\w+)>", text or "")
    if m:
        import struct
        bits, elem = int(m.group(1), 16), m.group(2)
        if elem == "f32":
            return struct.unpack("<f", struct.pack("<I", bits))[0]
        if elem == "f64":
            return struct.unpack("<d", struct.pack("<Q", bits))[0]
        if elem == "f16":
            return struct.unpack("<e", struct.pack("<H", bits))[0]
        if elem == "bf16":
            return struct.unpack("<f", struct.pack("<I", bits << 16))[0]
    raise ValueError(f"execution packet: expected a splat constant, got {text!r}")


def plan_packet(packet) -> dict:
    """Recognise the packet's tile program.  Returns a dict with `kind`
    ("gemm", "attention", "reduce", "fill" or "copy"), the kernel-argument
    positions of each operand,
    the program parameters and `layouts_match` (whether the packet's MMA
    contracts are the ones the library kernel implements)."""
    pk = _load(packet)
    ops = pk["operations"]
    kernels = [o for o in ops if o["name"] == "frisk.kernel"]
    if len(kernels) != 1 or not kernels[0].get("region_args"):
        raise ValueError("execution packet: expected exactly one frisk.kernel")
    args = kernels[0]["region_args"][0]
    types = {v["id"]: v["type"] for v in pk["values"]}
    producer, alias, filled = {}, {}, {}
    for o in ops:
        for r in o["results"]:
            producer[r] = o
        if o["name"] in ("frisk.layout_view", "frisk.convert_layout"):
            alias[o["results"][0]] = o["operands"][0]
    def root(v):
        while v in alias:
            v = alias[v]
        return v
    for o in ops:
        if o["name"] == "frisk.copy":
            filled[root(o["operands"][1])] = root(o["operands"][0])
    def source_arg(v):
        r = root(v)
        seen = set()
        while r in filled and r not in seen:
            seen.add(r)
            r = root(filled[r])
        if r not in args:
            raise ValueError(f"execution packet: value {v} does not come from a kernel argument")
        return args.index(r)
    body = [o for o in ops if o["name"] not in _TRANSPARENT]
    names = [o["name"] for o in body]
    contract = lambda o: o["attrs"].get("frisk.mma_contract", "")
    if names == ["frisk.mma", "frisk.tile_store"]:
        mma, store = body
        if store["operands"][0] != mma["results"][0]:
            raise ValueError("execution packet: the stored value is not the MMA result")
        init = producer.get(mma["operands"][2])
        if not init or init["name"] != "arith.constant" or _splat(init["attrs"].get("value")) != 0.0:
            raise ValueError("execution packet: GEMM accumulator must start from a zero constant")
        # The packet is one workgroup tile product: the compiled kernel that
        # executes its contract (MFMA atom and wave grid) runs it.
        m, n = mma["attrs"]["m"], mma["attrs"]["n"]
        threads = int(mma["attrs"].get("frisk.execution_threads", 0))
        variant, why = variants.variant_for(contract(mma), m, n, threads)
        return {"kind": "gemm", "a": source_arg(mma["operands"][0]), "b": source_arg(mma["operands"][1]),
                "c": source_arg(store["operands"][1]),
                "trans_a": bool(mma["attrs"].get("trans_a", False)),
                "trans_b": bool(mma["attrs"].get("trans_b", False)),
                "m": m, "n": n, "k": mma["attrs"]["k"], "threads": threads,
                "contract": contract(mma), "variant": variant, "layouts_match": variant is not None,
                "mismatch": why, "arg_types": [types[a] for a in args]}
    if names == _ATTENTION:
        qk, mul, rmax, bmax, sub, ex, rsum, bsum, div, trunc, pv, store = body
        chain = [(mul, 0, qk), (rmax, 0, mul), (bmax, 0, rmax), (sub, 0, mul), (sub, 1, bmax),
                 (ex, 0, sub), (rsum, 0, ex), (bsum, 0, rsum), (div, 0, ex), (div, 1, bsum),
                 (trunc, 0, div), (store, 0, pv)]
        for user, idx, prod in chain:
            if root(user["operands"][idx]) != prod["results"][0]:
                raise ValueError(f"execution packet: {user['name']} operand {idx} is not the "
                                 f"{prod['name']} result")
        if root(pv["operands"][0]) != trunc["results"][0]:
            raise ValueError("execution packet: P.V must consume the truncated probabilities")
        if rmax["attrs"].get("kind") != "max" or rsum["attrs"].get("kind") != "sum" or \
                rmax["attrs"].get("dim") != 1 or rsum["attrs"].get("dim") != 1:
            raise ValueError("execution packet: attention reductions must be max / sum over keys")
        if not qk["attrs"].get("trans_b") or qk["attrs"].get("trans_a") or \
                pv["attrs"].get("trans_a") or pv["attrs"].get("trans_b"):
            raise ValueError("execution packet: attention expects K stored [keys, dims] and V [keys, dims]")
        scale_op = producer.get(mul["operands"][1])
        if not scale_op or scale_op["name"] != "arith.constant":
            raise ValueError("execution packet: the score scale must be a constant")
        head_dim = qk["attrs"]["k"]
        # The attention kernel computes S^T = K.Q^T with the 32x32x16 atom
        # (queries on lanes, whole query rows per wave) and needs head_dim
        # >= 32 for its O^T tiles.
        kernel_layout = "swapped = true" in contract(qk) and "32x32x16" in contract(qk)
        why = "" if kernel_layout and head_dim >= 32 else (
            "the attention kernel computes S^T = K.Q^T with 32x32x16 MFMAs and head_dim >= 32; "
            f"this packet's QK contract is {contract(qk)} at head_dim {head_dim}")
        return {"kind": "attention", "q": source_arg(qk["operands"][0]), "k": source_arg(qk["operands"][1]),
                "v": source_arg(pv["operands"][1]), "o": source_arg(store["operands"][1]),
                "scale": _splat(scale_op["attrs"].get("value")), "seq_q": qk["attrs"]["m"],
                "seq_k": qk["attrs"]["n"], "head_dim": head_dim,
                "contract": contract(qk), "layouts_match": bool(kernel_layout and head_dim >= 32),
                "mismatch": why, "arg_types": [types[a] for a in args]}
    values = {v["id"]: v for v in pk["values"]}
    if names in (["frisk.tile_load", "frisk.reduce_tensor", "frisk.tile_store"],
                 ["frisk.tile_load", "frisk.reduce_tensor", "arith.addf", "frisk.tile_store"],
                 ["frisk.tile_load", "frisk.reduce_tensor", "arith.maximumf", "frisk.tile_store"],
                 ["frisk.tile_load", "frisk.reduce_tensor", "arith.minimumf", "frisk.tile_store"]):
        return _plan_reduce(body, producer, values, source_arg, types, args, root)
    if names == ["frisk.tile_store"]:
        store = body[0]
        cst = producer.get(store["operands"][0])
        if not cst or cst["name"] != "arith.constant":
            raise ValueError("execution packet: a lone tile_store must store a constant")
        return {"kind": "fill", "dst": source_arg(store["operands"][1]),
                "value": _splat(cst["attrs"].get("value")), "arg_types": [types[a] for a in args]}
    if names == ["frisk.tile_load", "frisk.tile_store"]:
        load, store = body
        if store["operands"][0] != load["results"][0]:
            raise ValueError("execution packet: the stored tile is not the loaded one")
        return {"kind": "copy", "src": source_arg(load["operands"][0]),
                "dst": source_arg(store["operands"][1]), "arg_types": [types[a] for a in args]}
    raise ValueError("execution packet: not a GEMM, attention, reduction, fill or copy tile "
                     "program: " + ", ".join(names))


_MERGE = {"arith.addf": "sum", "arith.maximumf": "max", "arith.minimumf": "min"}


def leaf_order_of(fibers, logical, shape, dim):
    """Leaf order of a reduction packet: for every output, the reduced index
    of each fiber leaf (carrier -> logical element -> index along `dim`), in
    fiber order.  Returns None for ascending order, else the bit permutation
    (tree level j combines along index bit order[j]) shared by all fibers."""
    cols = shape[1] if len(shape) == 2 else 1
    extent = shape[dim]
    order = None
    for fiber in fibers:
        idx = [(logical[c] // cols) if dim == 0 else (logical[c] % cols) for c in fiber]
        if len(idx) != extent or extent & (extent - 1):
            raise ValueError("execution packet: a reduction fiber does not hold every index of a "
                             "power-of-two extent once")
        nb = extent.bit_length() - 1
        bits = []
        for j in range(nb):
            v = idx[1 << j] ^ idx[0]
            if v & (v - 1) or v == 0:
                raise ValueError("execution packet: reduction leaf order is not a permutation of "
                                 "index bits")
            bits.append(v.bit_length() - 1)
        if idx[0] != 0 or any(idx[p] != sum(((p >> j) & 1) << bits[j] for j in range(nb))
                              for p in range(extent)):
            raise ValueError("execution packet: reduction leaf order is not a permutation of "
                             "index bits")
        if order is not None and bits != order:
            raise ValueError("execution packet: reduction fibers use different leaf orders")
        order = bits
    return None if order == sorted(order or []) else order


def _plan_reduce(body, producer, values, source_arg, types, args, root):
    load, red = body[0], body[1]
    store = body[-1]
    if root(red["operands"][0]) != load["results"][0]:
        raise ValueError("execution packet: the reduction does not read the loaded tile")
    kind, dim = red["attrs"].get("kind"), red["attrs"].get("dim")
    if kind not in ("sum", "max", "min") or dim not in (0, 1):
        raise ValueError(f"execution packet: reduction kind {kind!r} along {dim!r}")
    init = None
    result = red["results"][0]
    if len(body) == 4:
        merge = body[2]
        if _MERGE[merge["name"]] != kind:
            raise ValueError(f"execution packet: {merge['name']} cannot merge a {kind} reduction")
        if root(merge["operands"][1]) != result:
            raise ValueError("execution packet: the merge must combine (old value, reduction)")
        cst = producer.get(root(merge["operands"][0]))
        if not cst or cst["name"] != "arith.constant":
            raise ValueError("execution packet: the merged old value must be a constant")
        init = _splat(cst["attrs"].get("value"))
        result = merge["results"][0]
    if root(store["operands"][0]) != result:
        raise ValueError("execution packet: the stored value is not the reduction")
    src_val = values[load["results"][0]]
    dist = src_val.get("distributed")
    fibers = red.get("attrs", {}).get("fibers", red.get("fibers"))
    if not dist or fibers is None:
        raise ValueError("execution packet: the reduction has no fibers or source layout")
    shape = [int(x) for x in re.findall(r"(\d+)x", src_val["type"].split("<", 1)[1])]
    order = leaf_order_of(fibers, dist["logical"], shape, dim)
    return {"kind": "reduce", "src": source_arg(load["operands"][0]),
            "dst": source_arg(store["operands"][1]), "reduce": kind, "dim": dim, "init": init,
            "leaf_order": order, "arg_types": [types[a] for a in args]}


def execute_packet(packet, tensors, *, stream=None, require_layout_match=False,
                   allow_layout_mismatch=None) -> dict:
    """Run the packet on the GPU with `tensors` bound to the kernel's
    arguments (in order).  Returns the plan that was executed.

    The rule is execute()'s: a GEMM packet runs on the kernel variant its MMA
    contract selects, an attention packet on the attention kernel with the
    waves of its launch contract; when no kernel executes the packet's
    contract (`layouts_match` False, `mismatch` says why) the library's own
    kernel runs on the same tensors (same mathematics, other register
    layouts), unless `require_layout_match`, which raises ValueError
    instead.  (`allow_layout_mismatch=False` is the older spelling of
    require_layout_match=True.)"""
    from . import runtime as rt
    from .executor import _device_cus
    if allow_layout_mismatch is False:
        require_layout_match = True
    plan = plan_packet(packet)
    if plan["kind"] in ("gemm", "attention") and not plan["layouts_match"] and require_layout_match:
        raise ValueError(f"execution packet: no kernel executes this {plan['kind']} packet's "
                         f"instruction contract ({plan['mismatch']}); without "
                         "require_layout_match the library's own kernel runs")
    tensors = list(tensors)
    if len(tensors) != len(plan["arg_types"]):
        raise ValueError(f"execution packet: kernel takes {len(plan['arg_types'])} arguments, "
                         f"got {len(tensors)}")
    for t, ty in zip(tensors, plan["arg_types"]):
        shape = [int(x) for x in re.findall(r"(\d+)x", ty.split("<", 1)[1])]
        if list(t.shape) != shape:
            raise ValueError(f"execution packet: argument of type {ty} bound to a tensor of shape "
                             f"{tuple(t.shape)}")
    if plan["kind"] == "gemm":
        a, b, c = tensors[plan["a"]], tensors[plan["b"]], tensors[plan["c"]]
        variant = plan["variant"]
        if variant is not None:
            try:  # the variant's conditions (alignment, pitches) on these tensors
                rt.gemm_plan(a, b, c, trans_a=plan["trans_a"], trans_b=plan["trans_b"],
                             variant=variant)
            except ValueError as e:
                if require_layout_match:
                    raise
                plan["mismatch"] = f"variant {variant} does not run on these tensors ({e})"
                plan["layouts_match"], variant = False, None
        rt.gemm(a, b, c, trans_a=plan["trans_a"], trans_b=plan["trans_b"], stream=stream,
                variant=variant)
    elif plan["kind"] == "reduce":
        dst = tensors[plan["dst"]]
        if plan["init"] is not None:
            rt.fill(dst, plan["init"], stream=stream)
        rt.reduce(tensors[plan["src"]], dst, plan["reduce"], axis=plan["dim"],
                  clear=plan["init"] is None, leaf_order=plan["leaf_order"], stream=stream)
    elif plan["kind"] == "fill":
        rt.fill(tensors[plan["dst"]], plan["value"], stream=stream)
    elif plan["kind"] == "copy":
        rt.copy(tensors[plan["src"]], tensors[plan["dst"]], stream=stream)
    else:
        q, k, v, o = (tensors[plan[n]] for n in ("q", "k", "v", "o"))
        view = lambda t: t.view(1, 1, *t.shape)
        plan["waves"] = _ir().frisk.attention_launch_plan(1, q.shape[0], q.shape[1], False,
                                                          _device_cus())["waves"]
        rt.attn_fwd(view(q), view(k), view(v), view(o), causal=False, sm_scale=plan["scale"],
                    stream=stream, waves=plan["waves"])
    return plan
