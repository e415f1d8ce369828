"""The textual IR parser (frisk_amd/ir/parse.cpp) on the CPU: every program
the builder makes prints back identically after parsing (raw, normalized
and with inferred layouts), parsed programs plan and lower like the
originals, and malformed input is located by line and column."""
import re

import pytest

import frisk_amd as F
from frisk_amd import executor as E
from tests import programs as P

ir = F._ir()

BUILDERS = {
    "tiled_gemm": lambda: P.tiled_gemm(256, 256, 256),
    "tiled_gemm_tt": lambda: P.tiled_gemm(256, 256, 256, trans_a=True, trans_b=True, k_scale=2),
    "whole_gemm": lambda: P.whole_gemm(64, 64, 64, clear=False),
    "attention": lambda: P.attention(1, 2, 256, 64),
    "attention_kt": lambda: P.attention(1, 2, 256, 64, k_transposed=True, staged=False),
    "attention_tensor_form": lambda: P.attention_tensor_form(M=64, N=64, D=16),
    "row_reduce": lambda: P.row_reduce(256, 64, init=float("-inf")),
    "col_reduce": lambda: P.col_reduce_tiles(100, 256),
    "cast": lambda: P.tiled_cast(128, 256, staged=True),
    "fill": lambda: P.tiled_fill(64, 128, -2.5),
    "gemm_then_cast": lambda: P.gemm_then_cast(64, 64, 64),
    "single_tile_reduce": lambda: P.single_tile_reduce(64, 64, kind="max", init=float("-inf")),
    "single_tile_fill": lambda: P.single_tile_fill(64, 64, value=0.1),
}


def text(module):
    return ir.frisk.print_module(module)


def roundtrip(module):
    t = text(module)
    parsed = F.parse_module(t)
    assert parsed.verify(), parsed.verify_diagnostic()
    assert text(parsed) == t
    return parsed


@pytest.mark.parametrize("name", sorted(BUILDERS))
def test_print_parse_print_is_identity(name):
    s, _ = BUILDERS[name]()
    roundtrip(s.module)


@pytest.mark.parametrize("name", ["single_tile_reduce", "single_tile_fill", "attention_tensor_form"])
def test_roundtrip_after_normalize_and_inference(name):
    s, _ = BUILDERS[name]()
    s.module.set_attr("frisk.legacy_semantics", s.builder.get_str_attr("tensor_v1"))
    s.module.set_attr("frisk.target", s.builder.get_str_attr("gfx950"))
    if name != "attention_tensor_form":
        F.frisk.normalize_layout_ir(s.module, "gfx950")
        roundtrip(s.module)
    assert F.frisk.infer_layouts(s.module)["status"] == "materialized"
    parsed = roundtrip(s.module)
    # The parsed module exports the same packet, up to frisk.mma attributes
    # at their declared defaults (trans_a = trans_b = false, policy Square):
    # the assembly elides them, the parser materializes them.
    assert canonical(F.frisk.export_execution(parsed)) == canonical(F.frisk.export_execution(s.module))


def canonical(packet: str):
    import json
    pk = json.loads(packet)
    defaults = {"trans_a": False, "trans_b": False, "policy": "#frisk.gemm_warp_policy<Square>"}
    for op in pk["operations"]:
        if op["name"] == "frisk.mma":
            for k, v in defaults.items():
                if op["attrs"].get(k, v) == v:
                    op["attrs"].pop(k, None)
    return pk


@pytest.mark.parametrize("name", ["tiled_gemm", "attention", "row_reduce", "cast", "gemm_then_cast"])
def test_parsed_programs_plan_like_the_originals(name):
    s, _ = BUILDERS[name]()
    kernel = re.search(r"frisk.kernel @(\w+)", text(s.module)).group(1)
    a, b = E.plan(s.module, kernel), E.plan(F.parse_module(text(s.module)), kernel)
    if hasattr(a, "steps"):
        assert a.steps == b.steps and {k: (v.shape, v.elem, v.arg, v.alias) for k, v in a.bufs.items()} \
            == {k: (v.shape, v.elem, v.arg, v.alias) for k, v in b.bufs.items()}
    else:
        assert a == b


def test_inference_on_parsed_text_matches_the_builder():
    s, _ = P.attention_tensor_form(M=128, N=64, D=64, dtype="bf16", threads=256)
    s.module.set_attr("frisk.target", s.builder.get_str_attr("gfx950"))
    parsed = F.parse_module(text(s.module))
    r1, r2 = F.frisk.infer_layouts(s.module), F.frisk.infer_layouts(parsed)
    assert r1["assignments"] == r2["assignments"] and r1["cost"] == r2["cost"]
    assert text(parsed) == text(s.module)


def test_generic_form_with_regions_and_bare_operations():
    src = '''
      func.func @f(%a: tensor<4xf32>) -> tensor<4xf32> {
        %r = "test.wrap"(%a) ({
        ^bb0(%x: tensor<4xf32>):
          "test.yield"(%x) : (tensor<4xf32>) -> ()
        }) {tag = "w", n = 3 : i64} : (tensor<4xf32>) -> (tensor<4xf32>)
        return %r : tensor<4xf32>
      }'''
    m = F.parse_module(src)
    t = text(m)
    assert '"test.wrap"(%arg0) ({' in t and "^bb0(%arg1: tensor<4xf32>):" in t
    assert 'n = 3 : i64, tag = "w"' in t  # attributes are kept sorted
    assert text(F.parse_module(t)) == t


@pytest.mark.parametrize("src,where,msg", [
    ("module {\n  %0 = arith.addf %x, %y : f32\n}", "2:19", "use of undefined value %x"),
    ("module {\n  frisk.nope\n}", "2:3", "unknown operation 'frisk.nope'"),
    ("module {\n  %c = arith.constant 1 : index\n  %c = arith.constant 2 : index\n}", "3:3",
     "redefinition of %c"),
    ("module { %0 = arith.constant dense<1.0> : memref<4xf32> }", "1:", "dense attribute needs a tensor type"),
    ("module {\n  frisk.kernel @k(memref<4xf32, 1>) {\n  }\n}", "", "entry block arguments do not match"),
    ("module { %a = memref.alloc() : memref<4xq32> }", "1:", "expected"),
])
def test_malformed_input_is_located(src, where, msg):
    with pytest.raises(ValueError, match=re.escape(msg)) as e:
        F.parse_module(src)
    assert str(e.value).startswith(where), str(e.value)
