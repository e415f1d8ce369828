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
  frisk_attn_fwd with the packet's scale.

The packet's distributed layouts describe how the solver would place the
tile; the kernels use their own fixed layouts, and `plan_packet` reports
whether the two agree (for attention the kernel computes S^T = K.Q^T with
32x32x16 MFMAs and queries on lanes; see frisk_amd/csrc/attn.h).
"""
from __future__ import annotations

import json
import re
from typing import Any

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
    m = re.match(r"dense<([-+0-9.eEinfa]+)>", text or "")
    if not m:
        raise ValueError(f"execution packet: expected a splat constant, got {text!r}")
    return float(m.group(1))


def plan_packet(packet) -> dict:
    """Recognise the packet's tile program.  Returns a dict with `kind`
    ("gemm" or "attention"), the kernel-argument positions of each operand,
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
        return {"kind": "gemm", "a": source_arg(mma["operands"][0]), "b": source_arg(mma["operands"][1]),
                "c": source_arg(store["operands"][1]),
                "trans_a": bool(mma["attrs"].get("trans_a", False)),
                "trans_b": bool(mma["attrs"].get("trans_b", False)),
                "m": mma["attrs"]["m"], "n": mma["attrs"]["n"], "k": mma["attrs"]["k"],
                "contract": contract(mma), "layouts_match": True,
                "arg_types": [types[a] for a in args]}
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
        kernel_layout = "swapped = true" in contract(qk) and "32x32x16" in contract(qk)
        return {"kind": "attention", "q": source_arg(qk["operands"][0]), "k": source_arg(qk["operands"][1]),
                "v": source_arg(pv["operands"][1]), "o": source_arg(store["operands"][1]),
                "scale": _splat(scale_op["attrs"].get("value")), "seq_q": qk["attrs"]["m"],
                "seq_k": qk["attrs"]["n"], "head_dim": head_dim,
                "contract": contract(qk), "layouts_match": bool(kernel_layout and head_dim >= 32),
                "arg_types": [types[a] for a in args]}
    raise ValueError("execution packet: not a GEMM or attention tile program: " + ", ".join(names))


def execute_packet(packet, tensors, *, stream=None) -> dict:
    """Run the packet on the GPU with `tensors` bound to the kernel's
    arguments (in order).  Returns the plan that was executed."""
    from . import runtime as rt
    plan = plan_packet(packet)
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
        rt.gemm(tensors[plan["a"]], tensors[plan["b"]], tensors[plan["c"]], trans_a=plan["trans_a"],
                trans_b=plan["trans_b"], stream=stream)
    else:
        q, k, v, o = (tensors[plan[n]] for n in ("q", "k", "v", "o"))
        view = lambda t: t.view(1, 1, *t.shape)
        rt.attn_fwd(view(q), view(k), view(v), view(o), causal=False, sm_scale=plan["scale"],
                    stream=stream)
    return plan
